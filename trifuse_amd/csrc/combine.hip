// Weighted combine and small elementwise kernels.
//
// The reference combines the K expert outputs of a token with the routing
// gates and adds the residual (MLXNativeGraniteMoEPrefill.h:688-701, kernel
// text :54-70). Both combines sum the K routes of a token in k order in fp32,
// scale by the residual multiplier, add the residual and round once to bf16:
// combine_sorted takes rows the decode down projection already multiplied by
// their gates (fp32), combine_rows takes the prefill path's bf16 expert
// outputs and applies the gates itself.
#include "tfm_device.h"
#include "tfm_internal.h"

namespace tfm {

// 8 columns per thread; H % 8 == 0. For K <= KMAX every route's row index and
// then every row is requested before the first is used (rows of bad routes
// read row 0 and are dropped by a select), so a thread waits for memory
// twice rather than twice per route; larger K takes the plain loop.
template <int KMAX, bool F16>
__global__ __launch_bounds__(256) void combine_sorted_kernel(const float* __restrict__ P,
                                                             const int32_t* __restrict__ inverse,
                                                             const int32_t* __restrict__ n_valid,
                                                             int T, int K, int H,
                                                             const uint16_t* __restrict__ residual,
                                                             float rmul, uint16_t* __restrict__ y) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int per_row = H / 8;
  if (i >= (int64_t)T * per_row) return;
  const int t = (int)(i / per_row), c = (int)(i % per_row) * 8;
  float s[8];
#pragma unroll
  for (int v = 0; v < 8; ++v) s[v] = 0.0f;
  const int nv = *n_valid;
  if (K <= KMAX) {
    int row[KMAX];
#pragma unroll
    for (int k = 0; k < KMAX; ++k) row[k] = k < K ? inverse[(int64_t)t * K + k] : nv;
    float4 a[KMAX], b[KMAX];
#pragma unroll
    for (int k = 0; k < KMAX; ++k) {
      const int64_t r = row[k] < nv ? row[k] : 0;
      const float4* p = reinterpret_cast<const float4*>(P + r * H + c);
      a[k] = p[0];
      b[k] = p[1];
    }
#pragma unroll
    for (int k = 0; k < KMAX; ++k) {
      const bool on = row[k] < nv;
      s[0] = on ? s[0] + a[k].x : s[0]; s[1] = on ? s[1] + a[k].y : s[1];
      s[2] = on ? s[2] + a[k].z : s[2]; s[3] = on ? s[3] + a[k].w : s[3];
      s[4] = on ? s[4] + b[k].x : s[4]; s[5] = on ? s[5] + b[k].y : s[5];
      s[6] = on ? s[6] + b[k].z : s[6]; s[7] = on ? s[7] + b[k].w : s[7];
    }
  } else {
    for (int k = 0; k < K; ++k) {
      const int64_t row = inverse[(int64_t)t * K + k];
      if (row >= nv) continue;
      const float4* p = reinterpret_cast<const float4*>(P + row * H + c);
      const float4 a = p[0], b = p[1];
      s[0] += a.x; s[1] += a.y; s[2] += a.z; s[3] += a.w;
      s[4] += b.x; s[5] += b.y; s[6] += b.z; s[7] += b.w;
    }
  }
  float r[8];
  if (residual) {
    const uint4 rv = *reinterpret_cast<const uint4*>(residual + (int64_t)t * H + c);
    r[0] = lo_st<F16>(rv.x); r[1] = hi_st<F16>(rv.x); r[2] = lo_st<F16>(rv.y); r[3] = hi_st<F16>(rv.y);
    r[4] = lo_st<F16>(rv.z); r[5] = hi_st<F16>(rv.z); r[6] = lo_st<F16>(rv.w); r[7] = hi_st<F16>(rv.w);
  } else {
#pragma unroll
    for (int v = 0; v < 8; ++v) r[v] = 0.0f;
  }
  // y = bf16(fma(rm, sum, residual)), the rounding the fused small-batch
  // decode kernel (dstream.hip) reproduces.
  uint4 o;
  o.x = pack_st2<F16>(__builtin_fmaf(rmul, s[0], r[0]), __builtin_fmaf(rmul, s[1], r[1]));
  o.y = pack_st2<F16>(__builtin_fmaf(rmul, s[2], r[2]), __builtin_fmaf(rmul, s[3], r[3]));
  o.z = pack_st2<F16>(__builtin_fmaf(rmul, s[4], r[4]), __builtin_fmaf(rmul, s[5], r[5]));
  o.w = pack_st2<F16>(__builtin_fmaf(rmul, s[6], r[6]), __builtin_fmaf(rmul, s[7], r[7]));
  *reinterpret_cast<uint4*>(y + (int64_t)t * H + c) = o;
}

void launch_combine_sorted(bool f16, const float* P, const int32_t* inverse, const int32_t* n_valid, int T,
                           int K, int H, const uint16_t* residual, float rmul, uint16_t* y,
                           hipStream_t s) {
  if (T <= 0) return;
  const int64_t n = (int64_t)T * (H / 8);
  const unsigned blocks = (unsigned)((n + 255) / 256);
  if (f16)
    tfm_launch(combine_sorted_kernel<8, true>, blocks, 256, 0, s, P, inverse, n_valid, T, K, H, residual, rmul, y);
  else
    tfm_launch(combine_sorted_kernel<8, false>, blocks, 256, 0, s, P, inverse, n_valid, T, K, H, residual, rmul, y);
  check_hip(hipGetLastError(), "combine launch");
}

// 8 columns per thread; H % 8 == 0. Y rows are expert outputs in the storage
// dtype (bf16, or half when F16; the
// reference's per-route gather_qmm output, MLXNativeGraniteMoEPrefill.h:684),
// weighted by the fp32 gate and summed in k order. For K <= KMAX every
// route's row index and gate, then every row, are requested before the first
// is used (bad routes read row 0 and are dropped by a select), as in
// combine_sorted_kernel; larger K takes the plain loop.
template <int KMAX, bool F16>
__global__ __launch_bounds__(256) void combine_rows_kernel(const uint16_t* __restrict__ Y,
                                                           const int32_t* __restrict__ inverse,
                                                           const int32_t* __restrict__ n_valid,
                                                           const float* __restrict__ gates,
                                                           int T, int K, int H,
                                                           const uint16_t* __restrict__ residual,
                                                           float rmul, uint16_t* __restrict__ y) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int per_row = H / 8;
  if (i >= (int64_t)T * per_row) return;
  const int t = (int)(i / per_row), c = (int)(i % per_row) * 8;
  float s[8];
#pragma unroll
  for (int v = 0; v < 8; ++v) s[v] = 0.0f;
  const int nv = *n_valid;
  auto add = [&](float gw, const uint4& a, bool on) {
    s[0] = on ? __builtin_fmaf(gw, lo_st<F16>(a.x), s[0]) : s[0];
    s[1] = on ? __builtin_fmaf(gw, hi_st<F16>(a.x), s[1]) : s[1];
    s[2] = on ? __builtin_fmaf(gw, lo_st<F16>(a.y), s[2]) : s[2];
    s[3] = on ? __builtin_fmaf(gw, hi_st<F16>(a.y), s[3]) : s[3];
    s[4] = on ? __builtin_fmaf(gw, lo_st<F16>(a.z), s[4]) : s[4];
    s[5] = on ? __builtin_fmaf(gw, hi_st<F16>(a.z), s[5]) : s[5];
    s[6] = on ? __builtin_fmaf(gw, lo_st<F16>(a.w), s[6]) : s[6];
    s[7] = on ? __builtin_fmaf(gw, hi_st<F16>(a.w), s[7]) : s[7];
  };
  if (K <= KMAX) {
    int row[KMAX];
    float gw[KMAX];
#pragma unroll
    for (int k = 0; k < KMAX; ++k) {
      row[k] = k < K ? inverse[(int64_t)t * K + k] : nv;
      gw[k] = k < K ? gates[(int64_t)t * K + k] : 0.0f;
    }
    uint4 a[KMAX];
#pragma unroll
    for (int k = 0; k < KMAX; ++k) {
      const int64_t r = row[k] < nv ? row[k] : 0;
      a[k] = *reinterpret_cast<const uint4*>(Y + r * H + c);
    }
#pragma unroll
    for (int k = 0; k < KMAX; ++k) add(gw[k], a[k], row[k] < nv);
  } else {
    for (int k = 0; k < K; ++k) {
      const int64_t f = (int64_t)t * K + k;
      const int64_t row = inverse[f];
      if (row >= nv) continue;
      add(gates[f], *reinterpret_cast<const uint4*>(Y + row * H + c), true);
    }
  }
  float r[8];
  if (residual) {
    const uint4 rv = *reinterpret_cast<const uint4*>(residual + (int64_t)t * H + c);
    r[0] = lo_st<F16>(rv.x); r[1] = hi_st<F16>(rv.x); r[2] = lo_st<F16>(rv.y); r[3] = hi_st<F16>(rv.y);
    r[4] = lo_st<F16>(rv.z); r[5] = hi_st<F16>(rv.z); r[6] = lo_st<F16>(rv.w); r[7] = hi_st<F16>(rv.w);
  } else {
#pragma unroll
    for (int v = 0; v < 8; ++v) r[v] = 0.0f;
  }
  // y = st(fma(rm, sum, residual)), the rounding the fused small-batch
  // decode kernel (dstream.hip) reproduces.
  uint4 o;
  o.x = pack_st2<F16>(__builtin_fmaf(rmul, s[0], r[0]), __builtin_fmaf(rmul, s[1], r[1]));
  o.y = pack_st2<F16>(__builtin_fmaf(rmul, s[2], r[2]), __builtin_fmaf(rmul, s[3], r[3]));
  o.z = pack_st2<F16>(__builtin_fmaf(rmul, s[4], r[4]), __builtin_fmaf(rmul, s[5], r[5]));
  o.w = pack_st2<F16>(__builtin_fmaf(rmul, s[6], r[6]), __builtin_fmaf(rmul, s[7], r[7]));
  *reinterpret_cast<uint4*>(y + (int64_t)t * H + c) = o;
}

void launch_combine_rows(bool f16, const uint16_t* Y, const int32_t* inverse, const int32_t* n_valid,
                         const float* gates, int T, int K, int H, const uint16_t* residual,
                         float rmul, uint16_t* y, hipStream_t s) {
  if (T <= 0) return;
  const int64_t n = (int64_t)T * (H / 8);
  const unsigned blocks = (unsigned)((n + 255) / 256);
  if (f16)
    tfm_launch(combine_rows_kernel<8, true>, blocks, 256, 0, s, Y, inverse, n_valid, gates, T, K, H, residual, rmul, y);
  else
    tfm_launch(combine_rows_kernel<8, false>, blocks, 256, 0, s, Y, inverse, n_valid, gates, T, K, H, residual, rmul, y);
  check_hip(hipGetLastError(), "combine launch");
}

template <bool F16>
__global__ void rows_to_st_kernel(const float* __restrict__ P, int64_t n, uint16_t* __restrict__ out) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) out[i] = f2st<F16>(P[i]);
}

// fp32 rows rounded to the storage dtype (bf16, or IEEE half when f16).
void launch_rows_to_st(bool f16, const float* P, int64_t rows, int H, uint16_t* out, hipStream_t s) {
  const int64_t n = rows * H;
  if (n <= 0) return;
  if (f16)
    rows_to_st_kernel<true><<<(unsigned)((n + 255) / 256), 256, 0, s>>>(P, n, out);
  else
    rows_to_st_kernel<false><<<(unsigned)((n + 255) / 256), 256, 0, s>>>(P, n, out);
  check_hip(hipGetLastError(), "rows_to_st launch");
}

__global__ void copy_i32_kernel(const int32_t* __restrict__ a, int32_t* __restrict__ b, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) b[i] = a[i];
}

void launch_copy_i32(const int32_t* src, int32_t* dst, int64_t n, hipStream_t s) {
  if (n <= 0) return;
  copy_i32_kernel<<<(unsigned)((n + 255) / 256), 256, 0, s>>>(src, dst, n);
  check_hip(hipGetLastError(), "copy launch");
}

}  // namespace tfm
