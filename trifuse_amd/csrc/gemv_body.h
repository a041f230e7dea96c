// Device pieces of the decode GEMV shared by the standalone gather_qmm GEMV
// and the fused decode kernels: x staging in dot2 pair order, nibble unpack,
// DPP row reductions and the per-expert row loop.
#pragma once

#include "tfm_device.h"
#include "tfm_internal.h"

namespace tfm {

enum GemvMode { kGateUp = 0, kPlain = 1, kScaled = 2 };

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a),
                                         __builtin_bit_cast(bf16x2_t, b), c, false);
}

// The same dot product on packed pairs of the storage dtype: bf16 pairs, or
// IEEE-half pairs (v_dot2_f32_f16) when F16.
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
template <bool F16>
__device__ __forceinline__ float dot2_st(uint32_t a, uint32_t b, float c) {
  if constexpr (F16)
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2_t, a), __builtin_bit_cast(f16x2_t, b), c, false);
  else
    return dot2(a, b, c);
}

// (1.0, 1.0) in the storage dtype, and the value of the exponent byte that
// unpack_word_st places above each code: a code q becomes base + q exactly
// (bf16 0x43qq = 128 + q, half 0x64qq = 1024 + q for q < 16).
__host__ __device__ constexpr uint32_t ones2(bool f16) { return f16 ? 0x3c003c00u : 0x3f803f80u; }
__host__ __device__ constexpr float code_base(bool f16) { return f16 ? 1024.0f : 128.0f; }

template <int CTRL>
__device__ __forceinline__ float dpp_add(float v) {
  const int s = __builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, false);
  return v + __int_as_float(s);
}


// x chunk of one route in the pair order of the unpacked nibbles:
// for each packed word i (elements 8i..8i+7) pairs (0,2) (4,6) (1,3) (5,7).
struct ChunkX {
  uint32_t p[16];
  float sum;
};

template <bool F16 = false>
__device__ __forceinline__ void load_x(const uint16_t* __restrict__ src, ChunkX& cx) {
  const uint4* p4 = reinterpret_cast<const uint4*>(src);
  const uint32_t ones = ones2(F16);  // (1.0, 1.0) in the storage dtype
  float sum = 0.0f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint4 v = p4[i];  // (x0,x1) (x2,x3) (x4,x5) (x6,x7) of word i
    cx.p[4 * i + 0] = __builtin_amdgcn_perm(v.y, v.x, 0x05040100u);  // (x0, x2)
    cx.p[4 * i + 1] = __builtin_amdgcn_perm(v.w, v.z, 0x05040100u);  // (x4, x6)
    cx.p[4 * i + 2] = __builtin_amdgcn_perm(v.y, v.x, 0x07060302u);  // (x1, x3)
    cx.p[4 * i + 3] = __builtin_amdgcn_perm(v.w, v.z, 0x07060302u);  // (x5, x7)
    sum = dot2_st<F16>(v.x, ones, sum);
    sum = dot2_st<F16>(v.y, ones, sum);
    sum = dot2_st<F16>(v.z, ones, sum);
    sum = dot2_st<F16>(v.w, ones, sum);
  }
  cx.sum = sum;
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

// unpack_word for the storage dtype: pairs of (base+q) in bf16 or half.
template <bool F16>
__device__ __forceinline__ void unpack_word_st(uint32_t w, uint32_t* q) {
  const uint32_t magic = F16 ? 0x64646464u : 0x43434343u;
  const uint32_t lo = w & 0x0f0f0f0fu, hi = (w >> 4) & 0x0f0f0f0fu;
  q[0] = __builtin_amdgcn_perm(magic, lo, 0x04010400u);
  q[1] = __builtin_amdgcn_perm(magic, lo, 0x04030402u);
  q[2] = __builtin_amdgcn_perm(magic, hi, 0x04010400u);
  q[3] = __builtin_amdgcn_perm(magic, hi, 0x04030402u);
}

// Raw weights of one row-chunk: 16 packed bytes plus the bf16 scale and bias
// of its group, converted only when used.
struct RawW {
  uint4 q;
  uint32_t s;
  uint32_t b;
};

// Sum over aligned groups of G lanes using DPP only. The total lands in the
// last lane of each group (G = 32, 64) or in every lane (G <= 16).
template <int G>
__device__ __forceinline__ float dpp_group_sum(float v) {
  if (G >= 2) v = dpp_add<0xb1>(v);   // quad_perm [1,0,3,2]
  if (G >= 4) v = dpp_add<0x4e>(v);   // quad_perm [2,3,0,1]
  if (G >= 8) v = dpp_add<0x141>(v);  // row_half_mirror
  if (G >= 16) v = dpp_add<0x140>(v); // row_mirror: every lane of a row holds the row sum
  if (G >= 32) {                      // row_bcast:15 into rows 1 and 3
    const int s = __builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x142, 0xa, 0xf, false);
    v = v + __int_as_float(s);
  }
  if (G >= 64) {                      // row_bcast:31 into rows 2 and 3
    const int s = __builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x143, 0xc, 0xf, false);
    v = v + __int_as_float(s);
  }
  return v;
}

template <int G>
__device__ __forceinline__ bool group_sum_lane(int lane) {
  return G >= 32 ? (lane % G) == G - 1 : (lane % G) == 0;
}

// Buffer resource over [base, base + bytes): raw buffer loads at offsets
// beyond `bytes` return zero.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}

constexpr int kGemvXB = 4;     // routes staged per LDS batch
// Row units (one row-load per wave each) per workgroup, all of one expert:
// many short workgroups in flight measured faster at decode shapes than
// fewer, longer ones (deeper register prefetch costs occupancy).
constexpr int kGemvUnits = 2;

// LDS of the row units: the staged x chunks of up to kGemvXB routes.
struct GemvLds {
  uint4 xs[kGemvXB][4][64];  // [route][quarter][chunk]: 16 pair-dwords per chunk
  float xsum[kGemvXB][64];
};

// Row units of one routed expert. The rows of an expert are cut into units
// of UR = 4 * (64 / LG) rows (one row-load per wave); the calling workgroup
// (4 waves) processes units [rc0, rc0 + NU) (those below N rows) for routes
// [j0, j1) of expert e of matrices wa (and wb for gate/up, NM = 2). Every
// row-load is issued before the x staging, so their memory latencies overlap
// each other and the staging's.
//   xrow(j)            row of x feeding route j
//   stage(jb, nb)      called by every thread before the batch barrier, to
//                      stage per-route data of routes [jb, jb+nb)
//   emit(j, t, n, a0, a1)  called by the lane holding row n's totals for route
//                      j (batch slot t); a1 = a0 unless NM = 2.
// Every thread of the workgroup must call it (it contains barriers).
template <int LG, int NM, int NU, bool F16, typename XRow, typename Stage, typename Emit>
__device__ __forceinline__ void gemv_units(GemvLds& L, const uint16_t* __restrict__ x, int kin, int N,
                                           const tfm_affine& wa, const tfm_affine& wb, int e, int j0,
                                           int j1, int rc0, XRow xrow, Stage stage, Emit emit) {
  constexpr int RPL = 64 / LG;
  constexpr int UR = 4 * RPL;
  const int nch = kin / 32;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int sub = lane / LG, ll = lane % LG;
  const bool lane_ok = ll < nch;
  const uint32_t qrow = (uint32_t)kin / 2, srow = (uint32_t)kin / 32;  // bytes per row

  __amdgpu_buffer_rsrc_t rq[NM], rs[NM], rb[NM];
#pragma unroll
  for (int m = 0; m < NM; ++m) {
    const tfm_affine& mm = m == 0 ? wa : wb;
    rq[m] = make_rsrc(reinterpret_cast<const char*>(mm.q) + (size_t)e * N * qrow, (uint32_t)N * qrow);
    rs[m] = make_rsrc(static_cast<const char*>(mm.scales) + (size_t)e * N * srow, (uint32_t)N * srow);
    rb[m] = make_rsrc(static_cast<const char*>(mm.biases) + (size_t)e * N * srow, (uint32_t)N * srow);
  }
  // Row of this lane in unit u: rc0*UR + u*UR + wave*RPL + sub. Lanes past the
  // row's chunks read far out of range (zeros); rows past N are out of range
  // of the expert's buffer (zeros).
  const int n0 = rc0 * UR + wave * RPL + sub;
  const uint32_t qoff0 = lane_ok ? (uint32_t)n0 * qrow + 16u * ll : 0x7ff00000u;
  const uint32_t soff0 = (uint32_t)n0 * srow + 2u * (ll >> 1);
  auto load = [&](int u, RawW (&w)[NM]) {
    const uint32_t qo = qoff0 + (uint32_t)(u * UR) * qrow;
    const uint32_t so = soff0 + (uint32_t)(u * UR) * srow;
#pragma unroll
    for (int m = 0; m < NM; ++m) {
      w[m].q = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rq[m], qo, 0, 0));
      w[m].s = __builtin_amdgcn_raw_buffer_load_b16(rs[m], so, 0, 0);
      w[m].b = __builtin_amdgcn_raw_buffer_load_b16(rb[m], so, 0, 0);
    }
  };

  for (int jb = j0; jb < j1; jb += kGemvXB) {
    const int nb = min(kGemvXB, j1 - jb);
    RawW w[NU][NM];
#pragma unroll
    for (int u = 0; u < NU; ++u) load(u, w[u]);
    if (jb != j0) __syncthreads();  // every wave is done with the previous staging
    for (int p = tid; p < nb * nch; p += 256) {
      const int t = p / nch, c = p % nch;
      ChunkX cx;
      load_x<F16>(x + xrow(jb + t) * kin + 32 * c, cx);
#pragma unroll
      for (int q = 0; q < 4; ++q)
        L.xs[t][q][c] = make_uint4(cx.p[4 * q], cx.p[4 * q + 1], cx.p[4 * q + 2], cx.p[4 * q + 3]);
      L.xsum[t][c] = cx.sum;
    }
    stage(jb, nb);
    __syncthreads();
#pragma unroll
    for (int u = 0; u < NU; ++u) {
      const RawW (&cur)[NM] = w[u];
      float sc[NM], cc[NM];
#pragma unroll
      for (int m = 0; m < NM; ++m) {
        sc[m] = st2f<F16>((uint16_t)cur[m].s);
        cc[m] = __builtin_fmaf(-code_base(F16), sc[m], st2f<F16>((uint16_t)cur[m].b));
      }
      // One packed word at a time: its (base+q) pairs for every matrix, then
      // their dot products with the staged x of every route of the batch.
      float d0[kGemvXB][NM], d1[kGemvXB][NM];
#pragma unroll
      for (int t = 0; t < kGemvXB; ++t)
#pragma unroll
        for (int m = 0; m < NM; ++m) d0[t][m] = d1[t][m] = 0.0f;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        uint32_t qp[NM][4];
#pragma unroll
        for (int m = 0; m < NM; ++m) unpack_word_st<F16>(word_of(cur[m].q, q), qp[m]);
#pragma unroll
        for (int t = 0; t < kGemvXB; ++t) {
          if (t < nb) {
            const uint4 v = L.xs[t][q][ll];
#pragma unroll
            for (int m = 0; m < NM; ++m) {
              d0[t][m] = dot2_st<F16>(qp[m][0], v.x, d0[t][m]);
              d1[t][m] = dot2_st<F16>(qp[m][1], v.y, d1[t][m]);
              d0[t][m] = dot2_st<F16>(qp[m][2], v.z, d0[t][m]);
              d1[t][m] = dot2_st<F16>(qp[m][3], v.w, d1[t][m]);
            }
          }
        }
      }
      const int n = n0 + u * UR;
#pragma unroll
      for (int t = 0; t < kGemvXB; ++t) {
        if (t < nb) {
          const float xsm = L.xsum[t][ll];
          float acc[NM];
#pragma unroll
          for (int m = 0; m < NM; ++m)
            // Lanes past the row's chunks (kin < 32 * LG) contribute nothing;
            // their staged x is stale, so they are masked rather than
            // multiplied by 0.
            acc[m] = dpp_group_sum<LG>(lane_ok ? __builtin_fmaf(sc[m], d0[t][m] + d1[t][m], cc[m] * xsm) : 0.0f);
          if (group_sum_lane<LG>(lane) && n < N) emit(jb + t, t, n, acc[0], acc[NM - 1]);
        }
      }
    }
  }
}

}  // namespace tfm
