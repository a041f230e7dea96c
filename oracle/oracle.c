/*
 * CPU oracle for the TriFuse MoE feed-forward path: exact (bit-defined) parts.
 *
 * TEST INFRASTRUCTURE ONLY: loaded by tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py, never by the product library.
 *
 * Built with -ffp-contract=off: every fused multiply-add below is an explicit
 * fmaf(), so the arithmetic order is exactly what is written.
 */
#include "oracle.h"

#include <float.h>
#include <math.h>
#include <stdlib.h>
#include <string.h>

float orc_bf16_to_f32(uint16_t h) {
  uint32_t u = (uint32_t)h << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

uint16_t orc_f32_to_bf16(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x0040u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

/* IEEE half: exact widening; narrowing rounds to nearest even with subnormal
 * results, overflow to infinity (|f| >= 65520) and quiet NaN. */
float orc_f16_to_f32(uint16_t h) {
  const int e = (h >> 10) & 0x1f, m = h & 0x3ff;
  float v;
  if (e == 0x1f) v = m ? NAN : INFINITY;
  else if (e == 0) v = ldexpf((float)m, -24);
  else v = ldexpf((float)(m | 0x400), e - 25);
  return (h & 0x8000) ? -v : v;
}

uint16_t orc_f32_to_f16(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  const uint32_t sign = (u >> 16) & 0x8000u, a = u & 0x7fffffffu;
  if (a > 0x7f800000u) return (uint16_t)(sign | 0x7e00u | ((a >> 13) & 0x3ffu));
  if (a >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);
  if (a >= 0x38800000u) {
    const uint32_t r = a - 0x38000000u;
    return (uint16_t)(sign | ((r + 0xfffu + ((r >> 13) & 1u)) >> 13));
  }
  if (a <= 0x33000000u) return (uint16_t)sign;
  const uint32_t m = (a & 0x7fffffu) | 0x800000u;
  const int sh = 126 - (int)(a >> 23);
  uint32_t q = m >> sh;
  const uint32_t rem = m & ((1u << sh) - 1u), half = 1u << (sh - 1);
  q += (rem > half || (rem == half && (q & 1u))) ? 1u : 0u;
  return (uint16_t)(sign | q);
}

/* Storage dtype dt: 0 = bf16, 1 = IEEE half. */
static inline float st2f(int dt, uint16_t h) { return dt ? orc_f16_to_f32(h) : orc_bf16_to_f32(h); }
static inline uint16_t f2st(int dt, float f) { return dt ? orc_f32_to_f16(f) : orc_f32_to_bf16(f); }

void orc_f16_to_f32_array(const uint16_t* in, float* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = orc_f16_to_f32(in[i]);
}

void orc_f32_to_f16_array(const float* in, uint16_t* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = orc_f32_to_f16(in[i]);
}

void orc_bf16_to_f32_array(const uint16_t* in, float* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = orc_bf16_to_f32(in[i]);
}

void orc_f32_to_bf16_array(const float* in, uint16_t* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = orc_f32_to_bf16(in[i]);
}

/* Cody-Waite: x = n*ln2 + r with ln2 = LN2_HI + LN2_LO, LN2_HI = ln2 with its
 * low 16 significand bits cleared (0x3f317200), LN2_LO = fl(ln2 - LN2_HI).
 * e^r by Taylor's series to degree 7; the truncation term r^8/8! is below
 * 6e-9 relative on |r| <= ln2/2. Coefficients are fl(1/k!). */
float orc_expf(float x) {
  if (x != x) return x;
  if (x < -80.0f) return 0.0f;
  if (x > 88.0f) return INFINITY;
  const float n = rintf(x * 0x1.715476p+0f); /* fl(x * log2(e)) */
  float r = fmaf(-n, 0x1.62e4p-1f, x);       /* LN2_HI */
  r = fmaf(-n, 0x1.7f7d1cp-20f, r);          /* LN2_LO */
  float p = 0x1.a01a02p-13f;                 /* 1/7! */
  p = fmaf(p, r, 0x1.6c16c2p-10f);           /* 1/6! */
  p = fmaf(p, r, 0x1.111112p-7f);            /* 1/5! */
  p = fmaf(p, r, 0x1.555556p-5f);            /* 1/4! */
  p = fmaf(p, r, 0x1.555556p-3f);            /* 1/3! */
  p = fmaf(p, r, 0.5f);
  p = fmaf(p, r, 1.0f);
  p = fmaf(p, r, 1.0f);
  return ldexpf(p, (int)n);
}

void orc_expf_array(const float* in, float* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = orc_expf(in[i]);
}

/* Pairwise tree over 64 values in natural order: (0+1),(2+3)... then pairs of
 * pairs, in place; returns the root. */
static float tree64(float* v) {
  for (int w = 1; w < 64; w *= 2)
    for (int l = 0; l < 64; l += 2 * w) v[l] = v[l] + v[l + w];
  return v[0];
}

void orc_router_logits(const uint16_t* x, const uint16_t* w, const float* bias,
                       int T, int H, int E, uint16_t* logits) {
  const int c = H / 64;
  float lane[64];
  for (int t = 0; t < T; ++t) {
    const uint16_t* xr = x + (int64_t)t * H;
    for (int e = 0; e < E; ++e) {
      const uint16_t* wr = w + (int64_t)e * H;
      for (int l = 0; l < 64; ++l) {
        float s = 0.0f;
        for (int j = 0; j < c; ++j)
          s = fmaf(orc_bf16_to_f32(xr[l * c + j]), orc_bf16_to_f32(wr[l * c + j]), s);
        lane[l] = s;
      }
      float v = tree64(lane);
      if (bias) v = v + bias[e];
      logits[(int64_t)t * E + e] = orc_f32_to_bf16(v);
    }
  }
}

/* Affine-quantised router: the dense router's order over
 * w = st(fmaf(s, q, b)) (group 64), x, s, b and logits in storage dtype dt. */
void orc_router_logits_affine(const uint16_t* x, const uint32_t* q, const uint16_t* s,
                              const uint16_t* b, int bits, const float* bias, int T, int H, int E,
                              int dt, uint16_t* logits) {
  const int c = H / 64, per = 32 / bits;
  const uint32_t mask = (1u << bits) - 1u;
  float* w = (float*)malloc(sizeof(float) * (size_t)H);
  float lane[64];
  for (int e = 0; e < E; ++e) {
    const uint32_t* qr = q + (int64_t)e * (H / per);
    for (int k = 0; k < H; ++k) {
      const uint32_t code = (qr[k / per] >> (bits * (k % per))) & mask;
      const int64_t g = (int64_t)e * (H / 64) + k / 64;
      w[k] = st2f(dt, f2st(dt, fmaf(st2f(dt, s[g]), (float)code, st2f(dt, b[g]))));
    }
    for (int t = 0; t < T; ++t) {
      const uint16_t* xr = x + (int64_t)t * H;
      for (int l = 0; l < 64; ++l) {
        float acc = 0.0f;
        for (int j = 0; j < c; ++j) acc = fmaf(st2f(dt, xr[l * c + j]), w[l * c + j], acc);
        lane[l] = acc;
      }
      float v = tree64(lane);
      if (bias) v = v + bias[e];
      logits[(int64_t)t * E + e] = f2st(dt, v);
    }
  }
  free(w);
}

void orc_rmsnorm(const uint16_t* x, const uint16_t* w, float eps, int T, int H, int dt, uint16_t* out) {
  const int c = H / 64;
  float lane[64];
  for (int t = 0; t < T; ++t) {
    const uint16_t* xr = x + (int64_t)t * H;
    for (int l = 0; l < 64; ++l) {
      float s = 0.0f;
      for (int j = 0; j < c; ++j) {
        const float v = st2f(dt, xr[l * c + j]);
        s = fmaf(v, v, s);
      }
      lane[l] = s;
    }
    const float mean = tree64(lane) / (float)H;
    const float inv = 1.0f / sqrtf(mean + eps);
    for (int h = 0; h < H; ++h) {
      const float nx = st2f(dt, f2st(dt, st2f(dt, xr[h]) * inv));
      out[(int64_t)t * H + h] = f2st(dt, st2f(dt, w[h]) * nx);
    }
  }
}

/* Softmax normaliser in the reference's shape (MLXOLMoERouter.h:46-58):
 * four consecutive values summed in order, then a tree over the (up to 16)
 * four-value chunks; here the tree is the natural pairwise one, with absent
 * chunks contributing +0. Returns fl(1 / sum). ex has 64 entries. */
static float softmax_normaliser(const float* ex) {
  float chunk[64];
  for (int c = 0; c < 16; ++c) {
    float s = 0.0f;
    for (int i = 0; i < 4; ++i) s = s + ex[4 * c + i];
    chunk[c] = s;
  }
  for (int c = 16; c < 64; ++c) chunk[c] = 0.0f;
  return 1.0f / tree64(chunk);
}

/* exp(ld - max) of a 64-slot row whose absent slots are -inf
 * (MLXOLMoERouter.h:26-51): max starts at -FLT_MAX and skips NaN. */
static void softmax_exps(const float* ld, float* ex) {
  float maxval = -FLT_MAX;
  for (int i = 0; i < 64; ++i) maxval = maxval < ld[i] ? ld[i] : maxval;
  for (int i = 0; i < 64; ++i) ex[i] = orc_expf(ld[i] - maxval);
}

static void olmoe_probs(const uint16_t* row, int E, int dt, uint16_t* p) {
  float ld[64], ex[64];
  for (int i = 0; i < 64; ++i) ld[i] = i < E ? st2f(dt, row[i]) : -INFINITY;
  softmax_exps(ld, ex);
  const float norm = softmax_normaliser(ex);
  for (int i = 0; i < E; ++i) p[i] = f2st(dt, ex[i] * norm);
}

void orc_olmoe_softmax(const uint16_t* logits, int T, int E, int dt, uint16_t* probs) {
  for (int t = 0; t < T; ++t) olmoe_probs(logits + (int64_t)t * E, E, dt, probs + (int64_t)t * E);
}

void orc_route_olmoe(const uint16_t* logits, int T, int E, int K, int dt,
                     int32_t* idx, uint16_t* gates) {
  uint16_t p[64];
  for (int t = 0; t < T; ++t) {
    olmoe_probs(logits + (int64_t)t * E, E, dt, p);
    /* MLXOLMoERouter.h:65-83: stable descending rank, NaN last. */
    for (int i = 0; i < E; ++i) {
      const float v = st2f(dt, p[i]);
      const int vn = v != v;
      int rank = 0;
      for (int j = 0; j < E; ++j) {
        const float o = st2f(dt, p[j]);
        const int on = o != o;
        const int before = !on && (vn || o > v);
        const int equal = (on && vn) || (!on && !vn && o == v);
        rank += before || (equal && j < i);
      }
      if (rank < K) {
        idx[(int64_t)t * K + rank] = i;
        gates[(int64_t)t * K + rank] = p[i];
      }
    }
  }
}

void orc_route_granite(const uint16_t* logits, int T, int E, int K, int dt,
                       int32_t* idx, float* gates) {
  float v[64], sel[64], ld[64], ex[64];
  for (int t = 0; t < T; ++t) {
    const uint16_t* row = logits + (int64_t)t * E;
    for (int i = 0; i < E; ++i) v[i] = st2f(dt, row[i]);
    /* MLXNativeGraniteMoEPrefill.h:92-109: stable ascending rank, NaN last,
     * the top K ranks land in slots rank-(E-K). */
    for (int i = 0; i < E; ++i) {
      const int vn = v[i] != v[i];
      int rank = 0;
      for (int j = 0; j < E; ++j) {
        const int on = v[j] != v[j];
        const int less = !on && (vn || v[j] < v[i]);
        const int equal = (on && vn) || (!on && !vn && v[j] == v[i]);
        rank += less || (equal && j < i);
      }
      if (rank >= E - K) {
        sel[rank - (E - K)] = v[i];
        idx[(int64_t)t * K + rank - (E - K)] = i;
      }
    }
    /* MLXNativeGraniteMoEPrefill.h:112-149: fp32 softmax over the K slots. */
    for (int i = 0; i < 64; ++i) ld[i] = i < K ? sel[i] : -INFINITY;
    softmax_exps(ld, ex);
    const float norm = softmax_normaliser(ex);
    for (int i = 0; i < K; ++i) gates[(int64_t)t * K + i] = ex[i] * norm;
  }
}

int orc_group(const int32_t* idx, int64_t n, int E,
              int32_t* order, int32_t* inverse, int32_t* offsets) {
  int bad = 0;
  for (int64_t f = 0; f < n; ++f) bad += idx[f] < 0 || idx[f] >= E;
  if (bad) return bad;
  for (int e = 0; e <= E; ++e) offsets[e] = 0;
  for (int64_t f = 0; f < n; ++f) offsets[idx[f] + 1] += 1;
  for (int e = 0; e < E; ++e) offsets[e + 1] += offsets[e];
  int32_t* next = (int32_t*)malloc(sizeof(int32_t) * (size_t)(E > 0 ? E : 1));
  for (int e = 0; e < E; ++e) next[e] = offsets[e];
  for (int64_t f = 0; f < n; ++f) {
    const int32_t pos = next[idx[f]]++;
    order[pos] = (int32_t)f;
    inverse[f] = pos;
  }
  free(next);
  return 0;
}

void orc_dequant_f64(const uint32_t* q, const uint16_t* s, const uint16_t* b,
                     int N, int Kin, int group, int bits, int dt, double* w) {
  const int per = 32 / bits, words = Kin / per, groups = Kin / group;
  const uint32_t mask = (1u << bits) - 1u;
  for (int n = 0; n < N; ++n)
    for (int k = 0; k < Kin; ++k) {
      const uint32_t code = (q[(int64_t)n * words + k / per] >> (bits * (k % per))) & mask;
      const double sc = st2f(dt, s[(int64_t)n * groups + k / group]);
      const double bi = st2f(dt, b[(int64_t)n * groups + k / group]);
      w[(int64_t)n * Kin + k] = sc * (double)code + bi;
    }
}

void orc_gather_qmm_f64(const uint16_t* x, const int32_t* xrow, const int32_t* eid,
                        int rows, const uint32_t* q, const uint16_t* s, const uint16_t* b,
                        int N, int Kin, int group, int bits, int dt, double* out) {
  const int64_t qe = (int64_t)N * (Kin / (32 / bits)), se = (int64_t)N * (Kin / group);
  double* w = (double*)malloc(sizeof(double) * (size_t)N * (size_t)Kin);
  double* xf = (double*)malloc(sizeof(double) * (size_t)Kin);
  int last = -1;
  for (int r = 0; r < rows; ++r) {
    const int e = eid[r];
    if (e != last) {
      orc_dequant_f64(q + e * qe, s + e * se, b + e * se, N, Kin, group, bits, dt, w);
      last = e;
    }
    const uint16_t* xr = x + (int64_t)xrow[r] * Kin;
    for (int k = 0; k < Kin; ++k) xf[k] = st2f(dt, xr[k]);
    for (int n = 0; n < N; ++n) {
      double acc = 0.0;
      const double* wr = w + (int64_t)n * Kin;
      for (int k = 0; k < Kin; ++k) acc += xf[k] * wr[k];
      out[(int64_t)r * N + n] = acc;
    }
  }
  free(w);
  free(xf);
}

void orc_moe_reference(const uint16_t* x, const uint16_t* residual, float rm,
                       const int32_t* tokens, int ntok, int H, int I, int K,
                       const int32_t* idx, const float* gates, int group, int bits, int dt,
                       const uint32_t* gq, const uint16_t* gs, const uint16_t* gb,
                       const uint32_t* uq, const uint16_t* us, const uint16_t* ub,
                       const uint32_t* dq, const uint16_t* ds, const uint16_t* db,
                       double* out) {
  const int per = 32 / bits;
  const int64_t gu_e = (int64_t)I * (H / per), gu_s = (int64_t)I * (H / group);
  const int64_t d_e = (int64_t)H * (I / per), d_s = (int64_t)H * (I / group);
  double* wg = (double*)malloc(sizeof(double) * (size_t)I * (size_t)H);
  double* wu = (double*)malloc(sizeof(double) * (size_t)I * (size_t)H);
  double* wd = (double*)malloc(sizeof(double) * (size_t)H * (size_t)I);
  double* xf = (double*)malloc(sizeof(double) * (size_t)H);
  double* h = (double*)malloc(sizeof(double) * (size_t)I);
  int emax = -1;
  for (int i = 0; i < ntok; ++i)
    for (int k = 0; k < K; ++k) {
      const int e = idx[(int64_t)tokens[i] * K + k];
      emax = e > emax ? e : emax;
    }
  for (int64_t i = 0; i < (int64_t)ntok * H; ++i) out[i] = 0.0;
  /* Expert by expert so each expert is dequantised once; every token's K
   * contributions are then summed in k order below. */
  double* contrib = (double*)calloc((size_t)ntok * (size_t)K * (size_t)H, sizeof(double));
  for (int e = 0; e <= emax; ++e) {
    int used = 0;
    for (int i = 0; i < ntok && !used; ++i)
      for (int k = 0; k < K; ++k) used |= idx[(int64_t)tokens[i] * K + k] == e;
    if (!used) continue;
    orc_dequant_f64(gq + e * gu_e, gs + e * gu_s, gb + e * gu_s, I, H, group, bits, dt, wg);
    orc_dequant_f64(uq + e * gu_e, us + e * gu_s, ub + e * gu_s, I, H, group, bits, dt, wu);
    orc_dequant_f64(dq + e * d_e, ds + e * d_s, db + e * d_s, H, I, group, bits, dt, wd);
    for (int i = 0; i < ntok; ++i) {
      const int t = tokens[i];
      for (int k = 0; k < K; ++k) {
        if (idx[(int64_t)t * K + k] != e) continue;
        for (int c = 0; c < H; ++c) xf[c] = st2f(dt, x[(int64_t)t * H + c]);
        for (int n = 0; n < I; ++n) {
          double ag = 0.0, au = 0.0;
          const double* rg = wg + (int64_t)n * H;
          const double* ru = wu + (int64_t)n * H;
          for (int c = 0; c < H; ++c) { ag += xf[c] * rg[c]; au += xf[c] * ru[c]; }
          h[n] = ag / (1.0 + exp(-ag)) * au;
        }
        double* y = contrib + ((int64_t)i * K + k) * H;
        for (int c = 0; c < H; ++c) {
          double acc = 0.0;
          const double* rd = wd + (int64_t)c * I;
          for (int n = 0; n < I; ++n) acc += h[n] * rd[n];
          y[c] = acc;
        }
      }
    }
  }
  for (int i = 0; i < ntok; ++i) {
    const int t = tokens[i];
    double* o = out + (int64_t)i * H;
    for (int k = 0; k < K; ++k) {
      const double gate = gates[(int64_t)t * K + k];
      const double* y = contrib + ((int64_t)i * K + k) * H;
      for (int c = 0; c < H; ++c) o[c] += gate * y[c];
    }
    for (int c = 0; c < H; ++c) {
      o[c] *= (double)rm;
      if (residual) o[c] += st2f(dt, residual[(int64_t)t * H + c]);
    }
  }
  free(contrib); free(wg); free(wu); free(wd); free(xf); free(h);
}
