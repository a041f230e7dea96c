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

constexpr int kGemvXB = 4;  // routes staged per LDS batch
// Row-loads per wave: enough workgroups to fill the chip for a handful of
// routed experts, little per-workgroup setup relative to the weights read.
constexpr int kGemvRowLoads = 2;

// LDS of the row loop: the staged x chunks of up to kGemvXB routes.
struct GemvLds {
  uint4 xs[kGemvXB][4][64];  // [route][quarter][chunk]: 16 pair-dwords per chunk
  float xsum[kGemvXB][64];
};

// The row loop of one routed expert. The calling workgroup (4 waves) covers
// rows [wave_row0, wave_row0 + nit*RPL) per wave (wave_row0 already includes
// the wave), for routes [j0, j1) of expert `e` of matrices wa (and wb for
// gate/up, NM = 2).
//   xrow(j)            row of x feeding route j
//   stage(jb, nb)      called by every thread before the batch barrier, to
//                      stage per-route data of routes [jb, jb+nb)
//   emit(j, t, n, a0, a1)  called by the lane holding row n's totals for route
//                      j (batch slot t); a1 = a0 unless NM = 2.
// Every thread of the workgroup must call it (it contains barriers).
template <int LG, int NM, typename XRow, typename Stage, typename Emit>
__device__ __forceinline__ void gemv_expert_rows(GemvLds& L, const uint16_t* __restrict__ x, int kin,
                                                 int N, const tfm_affine& wa, const tfm_affine& wb,
                                                 int e, int j0, int j1, int nit, int wave_row0,
                                                 XRow xrow, Stage stage, Emit emit) {
  constexpr int RPL = 64 / LG;
  const int nch = kin / 32;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
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
  // Lanes past the row's chunks read far out of range (zeros).
  const uint32_t qoff0 = ll < nch ? (uint32_t)(wave_row0 + sub) * qrow + 16u * ll : 0x7ff00000u;
  const uint32_t soff0 = (uint32_t)(wave_row0 + sub) * srow + 2u * (ll >> 1);

  auto load = [&](int it, RawW (&w)[NM]) {
    const uint32_t qo = qoff0 + (uint32_t)(it * RPL) * qrow;
    const uint32_t so = soff0 + (uint32_t)(it * RPL) * srow;
#pragma unroll
    for (int m = 0; m < NM; ++m) {
      w[m].q = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rq[m], qo, 0, 0));
      w[m].s = __builtin_amdgcn_raw_buffer_load_b16(rs[m], so, 0, 0);
      w[m].b = __builtin_amdgcn_raw_buffer_load_b16(rb[m], so, 0, 0);
    }
  };

  for (int jb = j0; jb < j1; jb += kGemvXB) {
    const int nb = min(kGemvXB, j1 - jb);
    RawW cur[NM];
    if (nit > 0) load(0, cur);
    if (jb != j0) __syncthreads();
    for (int p = tid; p < nb * nch; p += 256) {
      const int t = p / nch, c = p % nch;
      ChunkX cx;
      load_x(x + xrow(jb + t) * kin + 32 * c, cx);
#pragma unroll
      for (int q = 0; q < 4; ++q)
        L.xs[t][q][c] = make_uint4(cx.p[4 * q], cx.p[4 * q + 1], cx.p[4 * q + 2], cx.p[4 * q + 3]);
      L.xsum[t][c] = cx.sum;
    }
    stage(jb, nb);
    __syncthreads();
#pragma unroll 1
    for (int it = 0; it < nit; ++it) {
      RawW nxt[NM];
      if (it + 1 < nit) load(it + 1, nxt);
      uint32_t qp[NM][16];
      float sc[NM], cc[NM];
#pragma unroll
      for (int m = 0; m < NM; ++m) {
        unpack_word(cur[m].q.x, &qp[m][0]);
        unpack_word(cur[m].q.y, &qp[m][4]);
        unpack_word(cur[m].q.z, &qp[m][8]);
        unpack_word(cur[m].q.w, &qp[m][12]);
        sc[m] = bf2f((uint16_t)cur[m].s);
        cc[m] = __builtin_fmaf(-128.0f, sc[m], bf2f((uint16_t)cur[m].b));
      }
      const int n = wave_row0 + it * RPL + sub;
#pragma unroll 1
      for (int t = 0; t < nb; ++t) {
        uint32_t xp[16];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const uint4 v = L.xs[t][q][ll];
          xp[4 * q] = v.x; xp[4 * q + 1] = v.y; xp[4 * q + 2] = v.z; xp[4 * q + 3] = v.w;
        }
        const float xsm = L.xsum[t][ll];
        float acc[NM];
#pragma unroll
        for (int m = 0; m < NM; ++m) {
          float d0 = 0.0f, d1 = 0.0f;
#pragma unroll
          for (int k = 0; k < 16; k += 2) {
            d0 = dot2(qp[m][k], xp[k], d0);
            d1 = dot2(qp[m][k + 1], xp[k + 1], d1);
          }
          // Lanes past the row's chunks (kin < 32 * LG) contribute nothing; their
          // staged x is stale, so they are masked rather than multiplied by 0.
          acc[m] = dpp_group_sum<LG>(lane_ok ? __builtin_fmaf(sc[m], d0 + d1, cc[m] * xsm) : 0.0f);
        }
        if (group_sum_lane<LG>(lane) && n < N) emit(jb + t, t, n, acc[0], acc[NM - 1]);
      }
#pragma unroll
      for (int m = 0; m < NM; ++m) cur[m] = nxt[m];
    }
  }
}

}  // namespace tfm
