/*
 * CPU oracle for the TriFuse MoE feed-forward path: the MLX-semantics CPU
 * block that serves as the host-core baseline.
 *
 * TEST INFRASTRUCTURE ONLY: loaded by tests/ and the cpu_baseline leg of
 * bench.py, never by the product library.
 *
 * It follows the op sequence of NativeGraniteMoEPrefill::moe
 * (MLXNativeGraniteMoEPrefill.h:627-702) and of the exported MoE.forward
 * (export_native_olmoe_target.py:200-218, export_native_granite_target.py:236-258):
 * router linear, route, stable grouping, gather_qmm up then gate, SwiGLU,
 * gather_qmm down, unsort, weighted sum, residual. Every op result is rounded
 * to bf16 (the activation dtype) and matmuls accumulate in fp32, as MLX does
 * for bf16 arrays. Expert rows are dequantised once per (expert, row) and
 * reused for every route of that expert; work is split over OpenMP threads.
 * Compiled with -ffast-math (no bit-exact claim is made for this file).
 */
#include "oracle.h"

#include <math.h>
#include <omp.h>
#include <stdlib.h>
#include <string.h>

static inline float bf(float v) { return orc_bf16_to_f32(orc_f32_to_bf16(v)); }

static void dequant_row(const uint32_t* q, const uint16_t* s, const uint16_t* b,
                        int Kin, int group, int bits, float* w) {
  const int per = 32 / bits;
  const uint32_t mask = (1u << bits) - 1u;
  for (int g = 0; g < Kin / group; ++g) {
    const float sc = orc_bf16_to_f32(s[g]), bi = orc_bf16_to_f32(b[g]);
    for (int k = g * group; k < (g + 1) * group; k += per) {
      const uint32_t word = q[k / per];
      for (int i = 0; i < per; ++i) w[k + i] = sc * (float)((word >> (bits * i)) & mask) + bi;
    }
  }
}

static inline float dot(const float* a, const float* b, int n) {
  float acc = 0.0f;
  for (int i = 0; i < n; ++i) acc += a[i] * b[i];
  return acc;
}

int orc_moe_block_cpu(const uint16_t* x, const uint16_t* residual, float rm,
                      int T, int H, int E, int K, int I, int group, int bits, int route_kind,
                      const uint16_t* router_w, const float* router_bias,
                      const uint32_t* gq, const uint16_t* gs, const uint16_t* gb,
                      const uint32_t* uq, const uint16_t* us, const uint16_t* ub,
                      const uint32_t* dq, const uint16_t* ds, const uint16_t* db,
                      int32_t* idx, float* gates, uint16_t* y, int threads) {
  if (threads > 0) omp_set_num_threads(threads);
  int used = 1;
  const int64_t R = (int64_t)T * K;
  uint16_t* logits = (uint16_t*)malloc(sizeof(uint16_t) * (size_t)T * (size_t)E);
  float* xf = (float*)malloc(sizeof(float) * (size_t)T * (size_t)H);
  int32_t* order = (int32_t*)malloc(sizeof(int32_t) * (size_t)R);
  int32_t* inverse = (int32_t*)malloc(sizeof(int32_t) * (size_t)R);
  int32_t* offsets = (int32_t*)malloc(sizeof(int32_t) * (size_t)(E + 1));
  float* hbuf = (float*)malloc(sizeof(float) * (size_t)R * (size_t)I);
  float* ybuf = (float*)malloc(sizeof(float) * (size_t)R * (size_t)H);

#pragma omp parallel
  {
#pragma omp single
    used = omp_get_num_threads();
#pragma omp for schedule(static)
    for (int t = 0; t < T; ++t) {
      orc_router_logits(x + (int64_t)t * H, router_w, router_bias, 1, H, E, logits + (int64_t)t * E);
      for (int c = 0; c < H; ++c) xf[(int64_t)t * H + c] = orc_bf16_to_f32(x[(int64_t)t * H + c]);
      if (route_kind == 0) {
        uint16_t g16[64];
        orc_route_olmoe(logits + (int64_t)t * E, 1, E, K, 0, idx + (int64_t)t * K, g16);
        for (int k = 0; k < K; ++k) gates[(int64_t)t * K + k] = orc_bf16_to_f32(g16[k]);
      } else {
        orc_route_granite(logits + (int64_t)t * E, 1, E, K, 0, idx + (int64_t)t * K, gates + (int64_t)t * K);
      }
    }
  }
  orc_group(idx, R, E, order, inverse, offsets);

  const int nb = 16; /* rows per work item */
  const int per = 32 / bits;
  const int64_t gu_e = (int64_t)I * (H / per), gu_s = (int64_t)I * (H / group);
  const int64_t d_e = (int64_t)H * (I / per), d_s = (int64_t)H * (I / group);
#pragma omp parallel
  {
    float* wg = (float*)malloc(sizeof(float) * (size_t)H);
    float* wu = (float*)malloc(sizeof(float) * (size_t)H);
    float* wd = (float*)malloc(sizeof(float) * (size_t)I);
    /* gather_qmm up and gate, then SwiGLU, per (expert, row block). */
#pragma omp for schedule(dynamic, 1) collapse(2)
    for (int e = 0; e < E; ++e)
      for (int n0 = 0; n0 < I; n0 += nb) {
        if (offsets[e] == offsets[e + 1]) continue;
        for (int n = n0; n < n0 + nb && n < I; ++n) {
          const int64_t qr = e * gu_e + (int64_t)n * (H / per), sr = e * gu_s + (int64_t)n * (H / group);
          dequant_row(gq + qr, gs + sr, gb + sr, H, group, bits, wg);
          dequant_row(uq + qr, us + sr, ub + sr, H, group, bits, wu);
          for (int j = offsets[e]; j < offsets[e + 1]; ++j) {
            const float* xr = xf + (int64_t)(order[j] / K) * H;
            const float up = bf(dot(xr, wu, H));
            const float gt = bf(dot(xr, wg, H));
            const float sg = bf(1.0f / (1.0f + expf(-gt)));
            hbuf[(int64_t)j * I + n] = bf(bf(gt * sg) * up);
          }
        }
      }
    /* gather_qmm down per (expert, row block). */
#pragma omp for schedule(dynamic, 1) collapse(2)
    for (int e = 0; e < E; ++e)
      for (int c0 = 0; c0 < H; c0 += nb) {
        if (offsets[e] == offsets[e + 1]) continue;
        for (int c = c0; c < c0 + nb && c < H; ++c) {
          const int64_t qr = e * d_e + (int64_t)c * (I / per), sr = e * d_s + (int64_t)c * (I / group);
          dequant_row(dq + qr, ds + sr, db + sr, I, group, bits, wd);
          for (int j = offsets[e]; j < offsets[e + 1]; ++j)
            ybuf[(int64_t)j * H + c] = bf(dot(hbuf + (int64_t)j * I, wd, I));
        }
      }
    free(wg); free(wu); free(wd);
    /* unsort, weighted sum over k, residual. */
#pragma omp for schedule(static)
    for (int t = 0; t < T; ++t)
      for (int c = 0; c < H; ++c) {
        float total = 0.0f, out;
        if (route_kind == 0) {
          for (int k = 0; k < K; ++k)
            total += bf(ybuf[(int64_t)inverse[(int64_t)t * K + k] * H + c] * gates[(int64_t)t * K + k]);
          out = bf(bf(total) * rm);
        } else {
          for (int k = 0; k < K; ++k)
            total += ybuf[(int64_t)inverse[(int64_t)t * K + k] * H + c] * gates[(int64_t)t * K + k];
          out = bf(bf(total) * rm);
        }
        if (residual) out = bf(orc_bf16_to_f32(residual[(int64_t)t * H + c]) + out);
        y[(int64_t)t * H + c] = orc_f32_to_bf16(out);
      }
  }
  free(logits); free(xf); free(order); free(inverse); free(offsets); free(hbuf); free(ybuf);
  return used;
}
