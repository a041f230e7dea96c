// Post-attention RMSNorm of the MoE block's input (MLXNativeGraniteMoEPrefill.h:
// 485: post = fast::rms_norm(h, post_norm, eps), then moe(post, h, ...)).
//
// One wave per row. The order is bit-defined, the same as the router linear:
// lane l sums x*x over its H/64 contiguous elements with sequential fused
// multiply-adds, then the pairwise xor tree over the 64 lanes; mean =
// sum / H; inv = 1 / sqrt(mean + eps) (correctly rounded division and
// square root); out = bf16(w * bf16(x * inv)), the normalised value rounded
// to the activation dtype before the weight multiply.
#include "tfm_device.h"
#include "tfm_internal.h"

namespace tfm {

__device__ __forceinline__ float readlane_f(float v, int l) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l));
}

template <int C, bool F16>
__global__ __launch_bounds__(256) void rmsnorm_kernel(const uint16_t* __restrict__ x,
                                                      const uint16_t* __restrict__ w, float eps,
                                                      int T, int H, uint16_t* __restrict__ out) {
  const int lane = threadIdx.x & 63;
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= T) return;  // whole wave
  const uint4* xs = reinterpret_cast<const uint4*>(x + (int64_t)t * H + lane * C);
  const uint4* ws = reinterpret_cast<const uint4*>(w + lane * C);
  uint4 xv[C / 8], wv[C / 8];
#pragma unroll
  for (int i = 0; i < C / 8; ++i) {
    xv[i] = xs[i];
    wv[i] = ws[i];
  }
  float s = 0.0f;
#pragma unroll
  for (int i = 0; i < C / 8; ++i) {
    const uint32_t u[4] = {xv[i].x, xv[i].y, xv[i].z, xv[i].w};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const float a = lo_st<F16>(u[k]), b = hi_st<F16>(u[k]);
      s = __builtin_fmaf(a, a, s);
      s = __builtin_fmaf(b, b, s);
    }
  }
  const float total = readlane_f(wave_tree_sum64(s), 63);
  const float mean = total / (float)H;
  const float inv = 1.0f / sqrtf(mean + eps);
  uint4* os = reinterpret_cast<uint4*>(out + (int64_t)t * H + lane * C);
#pragma unroll
  for (int i = 0; i < C / 8; ++i) {
    const uint32_t u[4] = {xv[i].x, xv[i].y, xv[i].z, xv[i].w};
    const uint32_t g[4] = {wv[i].x, wv[i].y, wv[i].z, wv[i].w};
    uint32_t o[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const float na = st2f<F16>(f2st<F16>(lo_st<F16>(u[k]) * inv)), nb = st2f<F16>(f2st<F16>(hi_st<F16>(u[k]) * inv));
      const uint32_t ra = f2st<F16>(lo_st<F16>(g[k]) * na), rb = f2st<F16>(hi_st<F16>(g[k]) * nb);
      o[k] = ra | (rb << 16);
    }
    os[i] = make_uint4(o[0], o[1], o[2], o[3]);
  }
}

// Any H % 64 == 0: the same arithmetic with scalar loads.
template <bool F16>
__global__ __launch_bounds__(256) void rmsnorm_generic(const uint16_t* __restrict__ x,
                                                       const uint16_t* __restrict__ w, float eps,
                                                       int T, int H, uint16_t* __restrict__ out) {
  const int lane = threadIdx.x & 63;
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= T) return;  // whole wave
  const int c = H / 64;
  const uint16_t* xr = x + (int64_t)t * H + lane * c;
  float s = 0.0f;
  for (int j = 0; j < c; ++j) {
    const float v = st2f<F16>(xr[j]);
    s = __builtin_fmaf(v, v, s);
  }
  const float total = readlane_f(wave_tree_sum64(s), 63);
  const float mean = total / (float)H;
  const float inv = 1.0f / sqrtf(mean + eps);
  uint16_t* orow = out + (int64_t)t * H + lane * c;
  for (int j = 0; j < c; ++j) {
    const float n = st2f<F16>(f2st<F16>(st2f<F16>(xr[j]) * inv));
    orow[j] = f2st<F16>(st2f<F16>(w[lane * c + j]) * n);
  }
}

template <bool F16>
static void rmsnorm_dt(const uint16_t* x, const uint16_t* w, float eps, int T, int H, uint16_t* out,
                       hipStream_t s) {
  const unsigned blocks = (unsigned)((T + 3) / 4);
  switch (H) {
    case 512: rmsnorm_kernel<8, F16><<<blocks, 256, 0, s>>>(x, w, eps, T, H, out); break;
    case 1024: rmsnorm_kernel<16, F16><<<blocks, 256, 0, s>>>(x, w, eps, T, H, out); break;
    case 1536: rmsnorm_kernel<24, F16><<<blocks, 256, 0, s>>>(x, w, eps, T, H, out); break;
    case 2048: rmsnorm_kernel<32, F16><<<blocks, 256, 0, s>>>(x, w, eps, T, H, out); break;
    case 3072: rmsnorm_kernel<48, F16><<<blocks, 256, 0, s>>>(x, w, eps, T, H, out); break;
    case 4096: rmsnorm_kernel<64, F16><<<blocks, 256, 0, s>>>(x, w, eps, T, H, out); break;
    default: rmsnorm_generic<F16><<<blocks, 256, 0, s>>>(x, w, eps, T, H, out); break;
  }
}

void launch_rmsnorm(bool f16, const uint16_t* x, const uint16_t* w, float eps, int T, int H,
                    uint16_t* out, hipStream_t s) {
  if (T <= 0) return;
  if (H % 64 != 0) fail(TFM_E_UNSUPPORTED, "rmsnorm: hidden width must be a multiple of 64");
  if (f16)
    rmsnorm_dt<true>(x, w, eps, T, H, out, s);
  else
    rmsnorm_dt<false>(x, w, eps, T, H, out, s);
  check_hip(hipGetLastError(), "rmsnorm launch");
}

}  // namespace tfm
