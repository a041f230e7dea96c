// Decode path: fused affine-4bit dequant GEMV over routed experts (no MFMA).
//
// A workgroup (4 waves) owns one routed expert (blockIdx.y indexes the
// ascending list of experts that received routes) and a contiguous block of
// output rows, so each packed weight byte is read from HBM once per call and
// applied to every route of its expert. The x rows of the expert's routes are
// staged once per workgroup in LDS. A lane owns one 32-element chunk of a row
// (one coalesced 16-byte load; LG lanes per row, 64/LG rows per load), and
// row partial sums are reduced across the LG lanes with DPP only.
//
// Arithmetic per 32-element chunk (which lies inside one 64-wide group):
//   sum_k x_k (s q_k + b) = s * sum_k x_k (128 + q_k) + (b - 128 s) * sum_k x_k.
// 128 + q is exact in bf16 and is built from a nibble with one byte permute
// (bf16 bits 0x43qq with qq = q), so the products run as v_dot2_f32_bf16 on
// (x_a, x_b) . (128+q_a, 128+q_b) pairs with fp32 accumulation; x is staged
// already permuted into the pair order of the unpacked nibbles, with its
// chunk sums. The kernel is VALU-bound at decode shapes (about 7 VALU ops to
// unpack 8 nibbles plus 4 dot2 per route), so instructions per weight byte are
// what the layout minimises.
#include <cstdlib>

#include "gemv_body.h"

namespace tfm {

// Standalone decode GEMV over grouped routes (gather_qmm and the MoE block
// given routes): workgroup (bx, a) (4 waves) streams NU row units of active
// expert a (blockIdx.y indexes the ascending active-expert list).
template <int LG, int MODE, bool F16, int NU = kGemvUnits>
__global__ __launch_bounds__(256) void gemv_kernel(const uint16_t* __restrict__ x, RowMap rm,
                                                   Grouping g, tfm_affine wa, tfm_affine wb,
                                                   int N, int kin, const float* __restrict__ gates,
                                                   void* __restrict__ out) {
  constexpr int NM = MODE == kGateUp ? 2 : 1;
  __shared__ GemvLds L;
  __shared__ float xgate[kGemvXB];
  __shared__ int xorow[kGemvXB];
  // Expert and route range of slot blockIdx.y: one read of the slot table
  // where the decode gate/up kernel wrote it, else active list then offsets.
  int e, j0, j1;
  if (g.slots) {
    const int4 sl = g.slots[blockIdx.y];
    if (sl.x < 0) return;
    e = sl.x;
    j0 = sl.y;
    j1 = sl.z;
  } else {
    if ((int)blockIdx.y >= grp_active_count(g)) return;
    e = grp_active_id(g, blockIdx.y);
    j0 = grp_offset(g, e);
    j1 = grp_offset(g, e + 1);
  }
  auto xrow = [&](int j) -> int64_t { return MODE == kScaled ? (int64_t)j : route_row(rm, j); };
  auto stage = [&](int jb, int nb) {
    const int t = threadIdx.x;
    if (t < nb) {
      if (MODE == kScaled)
        xgate[t] = g.gates_sorted ? g.gates_sorted[jb + t] : gates ? gates[route_flat(rm, jb + t)] : 1.0f;
      if (MODE == kPlain) xorow[t] = route_flat(rm, jb + t);
    }
  };
  auto emit = [&](int j, int t, int n, float a0, float a1) {
    if (MODE == kGateUp) {
      const float hv = a0 * __builtin_amdgcn_rcpf(1.0f + __expf(-a0)) * a1;
      static_cast<uint16_t*>(out)[(int64_t)j * N + n] = f2st<F16>(hv);
    } else if (MODE == kPlain) {
      static_cast<uint16_t*>(out)[(int64_t)xorow[t] * N + n] = f2st<F16>(a0);
    } else {
      static_cast<float*>(out)[(int64_t)j * N + n] = a0 * xgate[t];
    }
  };
  gemv_units<LG, NM, NU, F16>(L, x, kin, N, wa, wb, e, j0, j1, blockIdx.x * NU, xrow, stage,
                                 emit);
}

static int64_t gemv_cus() {
  static const int64_t cus = [] {
    int dev = 0, n = 0;
    if (hipGetDevice(&dev) != hipSuccess) return 256;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
      return 256;
    return n;
  }();
  return cus;
}

template <int MODE, bool F16>
static void dispatch_gemv(int Kin, const uint16_t* x, RowMap rm, const Grouping& g, int max_active,
                          const tfm_affine& wa, const tfm_affine& wb, int N, const float* gates,
                          void* out, hipStream_t s) {
  if (max_active <= 0 || N <= 0) return;
  if (Kin % 64 != 0 || Kin <= 0 || Kin > 2048)
    fail(TFM_E_UNSUPPORTED, "affine GEMV: input width must be a multiple of 64 up to 2048");
  const int nch = Kin / 32;
  // Plain products (gather_qmm, the dense linear) with fewer workgroups than
  // two per compute unit take one row unit per workgroup, twice the
  // workgroups: the dense 2048 x 2048 linear at one row 4.47 -> 4.06 us, the
  // 64 x 2048 router 3.2 -> 2.8 us. The MoE block's GEMVs have many
  // experts' workgroups and keep two units (one measured slower there).
#define TFM_GEMV_LAUNCH_NU(LGV, NUV)                                                        \
  {                                                                                         \
    const int ur = 4 * (64 / LGV), upe = (N + ur - 1) / ur;                                 \
    const dim3 grid((unsigned)((upe + NUV - 1) / NUV), (unsigned)max_active);               \
    tfm_launch(gemv_kernel<LGV, MODE, F16, NUV>, grid, 256, 0, s, x, rm, g, wa, wb, N, Kin, gates, out); \
  }
#define TFM_GEMV_LAUNCH(LGV)                                                                    \
  {                                                                                             \
    const int64_t ur = 4 * (64 / LGV), upe = (N + ur - 1) / ur;                                 \
    const bool one = MODE == kPlain &&                                                          \
                     (int64_t)max_active * ((upe + kGemvUnits - 1) / kGemvUnits) < 2 * gemv_cus(); \
    if (one) TFM_GEMV_LAUNCH_NU(LGV, 1)                                                         \
    else TFM_GEMV_LAUNCH_NU(LGV, kGemvUnits)                                                    \
  }
  if (nch <= 4) TFM_GEMV_LAUNCH(4)
  else if (nch <= 8) TFM_GEMV_LAUNCH(8)
  else if (nch <= 16) TFM_GEMV_LAUNCH(16)
  else if (nch <= 32) TFM_GEMV_LAUNCH(32)
  else TFM_GEMV_LAUNCH(64)
#undef TFM_GEMV_LAUNCH
#undef TFM_GEMV_LAUNCH_NU
  check_hip(hipGetLastError(), "gemv launch");
}

void launch_gemv_gateup(bool f16, const uint16_t* x, RowMap rm, const Grouping& g, int max_active,
                        int64_t routes, const tfm_affine& gate, const tfm_affine& up, int N,
                        int Kin, uint16_t* h, hipStream_t s) {
  (void)routes;
  if (f16)
    dispatch_gemv<kGateUp, true>(Kin, x, rm, g, max_active, gate, up, N, nullptr, h, s);
  else
    dispatch_gemv<kGateUp, false>(Kin, x, rm, g, max_active, gate, up, N, nullptr, h, s);
}

void launch_gemv_plain(bool f16, const uint16_t* x, RowMap rm, const Grouping& g, int max_active,
                       int64_t routes, const tfm_affine& w, int N, int Kin, uint16_t* out,
                       hipStream_t s) {
  (void)routes;
  if (f16)
    dispatch_gemv<kPlain, true>(Kin, x, rm, g, max_active, w, w, N, nullptr, out, s);
  else
    dispatch_gemv<kPlain, false>(Kin, x, rm, g, max_active, w, w, N, nullptr, out, s);
}

void launch_gemv_scaled(bool f16, const uint16_t* hsorted, const Grouping& g, int max_active,
                        int64_t routes, const tfm_affine& w, int N, int Kin, const float* gates,
                        float* P, hipStream_t s) {
  (void)routes;
  RowMap rm{g.order, nullptr, 1, 0, nullptr};
  if (f16)
    dispatch_gemv<kScaled, true>(Kin, hsorted, rm, g, max_active, w, w, N, gates, P, s);
  else
    dispatch_gemv<kScaled, false>(Kin, hsorted, rm, g, max_active, w, w, N, gates, P, s);
}

}  // namespace tfm
