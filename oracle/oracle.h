/*
 * CPU oracle for the TriFuse MoE feed-forward path.
 *
 * TEST INFRASTRUCTURE ONLY. Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load this library, and only as the checker
 * (or, for the baseline, as the thing timed on the host cores). The product
 * path (trifuse_amd, libtrifuse_moe.so) never links, loads or calls it.
 *
 * It restates the reference's algorithm for the MoE block:
 *   router linear -> route (OLMoE or Granite rules) -> stable grouping ->
 *   affine 4-bit group-quantized expert matmuls (gate/up, SwiGLU, down) ->
 *   weighted combine (+ residual).
 * Each function cites the reference file:line it follows.
 *
 * Storage: activations, router weights, scales and biases are 16-bit bit
 * patterns (uint16_t) of the storage dtype dt: 0 = bf16, 1 = IEEE half.
 * Packed weights are uint32 words of 32/bits LSB-first codes (8 nibbles for
 * 4-bit, 4 bytes for 8-bit).
 */
#ifndef TFM_ORACLE_H
#define TFM_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* bf16 <-> fp32, round to nearest even; NaN stays NaN (quiet). */
float orc_bf16_to_f32(uint16_t h);
uint16_t orc_f32_to_bf16(float f);
void orc_bf16_to_f32_array(const uint16_t* in, float* out, int64_t n);
void orc_f32_to_bf16_array(const float* in, uint16_t* out, int64_t n);

/* IEEE half <-> fp32: widening is exact; narrowing rounds to nearest even,
 * keeps subnormal results, overflows to infinity at |f| >= 65520 and keeps
 * NaN quiet. */
float orc_f16_to_f32(uint16_t h);
uint16_t orc_f32_to_f16(float f);
void orc_f16_to_f32_array(const uint16_t* in, float* out, int64_t n);
void orc_f32_to_f16_array(const float* in, uint16_t* out, int64_t n);

/* exp for the routing softmax: Cody-Waite reduction by ln2 (hi/lo split) and
 * the degree-7 Taylor polynomial of e^r on |r| <= ln2/2, Horner with fma.
 * x < -80 returns 0 so every softmax term stays a normal number. */
float orc_expf(float x);
void orc_expf_array(const float* in, float* out, int64_t n);

/* Router logits, dense bf16 router W[E,H]:
 *   logits[t,e] = bf16( tree64(lane sums) + bias[e] )
 * lane l (0..63) sums x*w over h in [l*c, l*c+c), c = H/64, sequential fma
 * from 0; tree64 is the pairwise tree over the 64 lane sums in natural order.
 * bias may be NULL. Requires H % 64 == 0.
 * Reference: MLXNativeGraniteMoEPrefill.h:539-541,631 (router linear whose
 * output is in the activation dtype). */
void orc_router_logits(const uint16_t* x, const uint16_t* w, const float* bias,
                       int T, int H, int E, uint16_t* logits);

/* Post-attention RMSNorm in the layer's dtype (MLXNativeGraniteMoEPrefill.h:
 * 485, fast::rms_norm(h, post_norm, eps)), with this build's bit-defined
 * order: lane l (0..63) sums x*x over h in [l*c, l*c+c), c = H/64,
 * sequential fma from 0; tree64 over the 64 lane sums; mean = fl(sum / H);
 * inv = fl(1 / fl(sqrt(mean + eps))); then
 *   out[t,h] = bf16( w[h] * bf16( x[t,h] * inv ) )
 * (the normalised value is rounded to the activation dtype before the
 * weight multiply, MLX's rms_norm rounding points). Requires H % 64 == 0. */
void orc_rmsnorm(const uint16_t* x, const uint16_t* w, float eps, int T, int H, int dt, uint16_t* out);

/* Router logits of the affine-quantised router (the exports' router Affine
 * module, native_affine_qmm(x, W, S, B, 64, bits): export_native_olmoe_target.py:
 * 166-167,200; export_native_granite_target.py:236-237): the dense router's
 * order above over w[e,h] = st(fmaf(s, q, b)), the dequantised weight rounded
 * to the storage dtype as native_affine_ops.py:29-36 does. Q [E, H*bits/32],
 * S/B [E, H/64]; x, S, B and logits in dtype dt. */
void orc_router_logits_affine(const uint16_t* x, const uint32_t* q, const uint16_t* s,
                              const uint16_t* b, int bits, const float* bias, int T, int H, int E,
                              int dt, uint16_t* logits);

/* OLMoE routing: fp32 softmax over E with probabilities rounded to the
 * storage dtype, then the K largest probabilities in descending order, ties
 * to the lower expert id, NaN last; gates are those probabilities, not
 * renormalised.
 * Reference: MLXOLMoERouter.h:19-84,116-119; native_affine_ops.py:128-146;
 * native_affine_lowering.py:85-108. E <= 64. */
void orc_route_olmoe(const uint16_t* logits, int T, int E, int K, int dt,
                     int32_t* idx, uint16_t* gates);

/* Full probability rows of the OLMoE softmax (for tests). */
void orc_olmoe_softmax(const uint16_t* logits, int T, int E, int dt, uint16_t* probs);

/* Granite routing: the K largest logits selected by a stable ascending rank
 * (ties: higher id selected at the boundary, NaN last), slots in ascending
 * logit order, gates = fp32 softmax over the K selected logits.
 * Reference: MLXNativeGraniteMoEPrefill.h:77-150,622-624;
 * native_affine_lowering.py:61-74; export_native_granite_target.py:238-240. */
void orc_route_granite(const uint16_t* logits, int T, int E, int K, int dt,
                       int32_t* idx, float* gates);

/* Stable grouping of the T*K flat routes by expert:
 *   order[pos] = flat route index, sorted by (expert asc, flat asc)
 *   inverse[flat] = pos, offsets[e] = first pos of expert e, offsets[E] = T*K.
 * Returns the number of out-of-range ids (0 when valid; outputs untouched
 * otherwise). Reference: MLXNativeGraniteMoEPrefill.h:666-684;
 * export_native_olmoe_target.py:206-210. */
int orc_group(const int32_t* idx, int64_t n, int E,
              int32_t* order, int32_t* inverse, int32_t* offsets);

/* Affine dequantisation w = s*q + b of one expert matrix Q[N,Kin*bits/32]
 * (32/bits codes per word, LSB first), S/B [N,Kin/g] in dtype dt to fp64
 * (exact for bf16 and half S/B). bits is 4 or 8. Reference:
 * native_affine_ops.py:29-36. */
void orc_dequant_f64(const uint32_t* q, const uint16_t* s, const uint16_t* b,
                     int N, int Kin, int group, int bits, int dt, double* w);

/* gather_qmm, transpose=true: out[r,n] = sum_k x[xrow[r],k] * W[eid[r]][n,k]
 * in fp64 from exact dequantised weights. Reference: native_affine_ops.py:55-63;
 * MLXNativeGraniteMoEPrefill.h:542-550. */
void orc_gather_qmm_f64(const uint16_t* x, const int32_t* xrow, const int32_t* eid,
                        int rows, const uint32_t* q, const uint16_t* s, const uint16_t* b,
                        int N, int Kin, int group, int bits, int dt, double* out);

/* Numeric reference of the MoE block for the listed tokens: fp64 accumulation
 * over exact dequantised weights, SwiGLU in fp64, weighted combine with the
 * given gates (fp32 values), y = residual + rm * sum_k gate_k * expert_k(x).
 * residual may be NULL. out is [ntok, H] fp64.
 * Reference: MLXNativeGraniteMoEPrefill.h:627-702 (moe). */
void orc_moe_reference(const uint16_t* x, const uint16_t* residual, float rm,
                       const int32_t* tokens, int ntok, int H, int I, int K,
                       const int32_t* idx, const float* gates, int group, int bits, int dt,
                       const uint32_t* gq, const uint16_t* gs, const uint16_t* gb,
                       const uint32_t* uq, const uint16_t* us, const uint16_t* ub,
                       const uint32_t* dq, const uint16_t* ds, const uint16_t* db,
                       double* out);

/* The MLX-semantics CPU block (the host-core baseline): the reference's op
 * sequence with a bf16 result at every op boundary and fp32 accumulation,
 * parallel over routes with OpenMP. route_kind 0 = OLMoE, 1 = Granite.
 * router_bias may be NULL. Writes idx/gates (gates as fp32 values) and
 * y [T,H] bf16. Returns the number of threads used. */
int orc_moe_block_cpu(const uint16_t* x, const uint16_t* residual, float rm,
                      int T, int H, int E, int K, int I, int group, int bits, int route_kind,
                      const uint16_t* router_w, const float* router_bias,
                      const uint32_t* gq, const uint16_t* gs, const uint16_t* gb,
                      const uint32_t* uq, const uint16_t* us, const uint16_t* ub,
                      const uint32_t* dq, const uint16_t* ds, const uint16_t* db,
                      int32_t* idx, float* gates, uint16_t* y, int threads);

#ifdef __cplusplus
}
#endif
#endif
