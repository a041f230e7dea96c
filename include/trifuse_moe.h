/*
 * trifuse_moe.h - C ABI of the MI355X (gfx950) MoE feed-forward library.
 *
 * The library replaces, for one GPU, the MoE feed-forward path of TriFuse's
 * ExecuTorch MLX overlay: router linear, routing (OLMoE or Granite rules),
 * token-to-expert grouping, MLX affine 4-bit or 8-bit group-64 expert matmuls
 * (gate/up -> SwiGLU -> down) and the weighted combine (+ residual).
 *
 * Conventions
 *  - Every pointer argument named x, q, scales, ... is a DEVICE pointer owned
 *    by the caller and borrowed for the call. Work is enqueued on `stream`
 *    (a hipStream_t; NULL = the default stream) and the call returns as soon
 *    as it is enqueued. Results are valid after the stream is synchronised.
 *  - No call allocates device memory after tfm_plan_create: scratch memory
 *    comes from the caller's workspace (size from the *_workspace_bytes call).
 *    The first 256 bytes of a workspace hold the device status word: zero
 *    them once when the workspace is allocated. Kernels only set status bits;
 *    they stay set across calls until tfm_status_word reads and clears them.
 *  - Every entry point returns an int status (TFM_OK == 0). No C++ exception
 *    crosses the ABI; tfm_last_error() returns the calling thread's message.
 *  - Affine weight layout (identical to MLX / TriFuse packs):
 *      Q      uint32 [E, N, Kin*bits/32], p = 32/bits codes per word, LSB first
 *      scales dtype  [E, N, Kin/group]
 *      biases dtype  [E, N, Kin/group]
 *      w[n,k] = scales[n,k/group] * ((Q[n,k/p] >> bits*(k%p)) & (2^bits-1)) + biases[n,k/group]
 *    (native_affine_ops.py:29-36). gate/up: N = I, Kin = H; down: N = H, Kin = I.
 *  - Matmuls are "transpose=true": y = x . w^T (native_affine_lowering.py:28-31).
 *  - Plans are immutable once created and may be shared by threads. Calls that
 *    share one workspace must be ordered on one stream.
 */
#ifndef TRIFUSE_MOE_H
#define TRIFUSE_MOE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes ---------------------------------------------------- */
#define TFM_OK 0
#define TFM_E_INVALID 1     /* bad argument, geometry or dtype            */
#define TFM_E_UNSUPPORTED 2 /* valid for the reference, not built here    */
#define TFM_E_WORKSPACE 3   /* workspace missing or too small             */
#define TFM_E_HIP 4         /* HIP runtime error (launch, device query)   */
#define TFM_E_DEVICE 5      /* device-side check failed (see tfm_status_word) */

/* ---- enums ----------------------------------------------------------- */
#define TFM_DTYPE_BF16 0 /* activations, scales and biases in bf16         */
#define TFM_DTYPE_F16 1  /* IEEE half: TriFuse's shipped packs; needs the
                            affine router                                 */

#define TFM_ROUTE_OLMOE 0   /* softmax over E, top-K probabilities         */
#define TFM_ROUTE_GRANITE 1 /* top-K logits, softmax over the K selected   */

#define TFM_ROUTER_DENSE 0  /* router weight dtype [E,H]                   */
#define TFM_ROUTER_AFFINE 1 /* affine-quantised router (group 64)          */

/* tfm_moe_forward / tfm_moe_experts flags */
#define TFM_FLAG_DETERMINISTIC 1u /* accepted for compatibility: every path reduces the K routes of a token in k order */

/* Bits of the device status word (tfm_status_word). */
#define TFM_STATUS_BAD_EXPERT_ID 1u /* an expert id outside [0, E) was seen   */
#define TFM_STATUS_BAD_ROW_INDEX 2u /* a token/row index outside x was seen   */

/* ---- plan ------------------------------------------------------------ */
/* Geometry of one MoE block; mirrors NativeModelConfig
 * (resident_prefill.h:18-42) and its admission (MLXNativeGraniteMoEPrefill.h:306-330). */
typedef struct tfm_geometry {
  int32_t hidden_size;       /* H: multiple of 64                        */
  int32_t intermediate_size; /* I: multiple of 64                        */
  int32_t num_experts;       /* E: 1..64                                 */
  int32_t experts_per_token; /* K: 1..E                                  */
  int32_t group_size;        /* 64                                       */
  int32_t bits;              /* 4 or 8 (8-bit: grouped GEMM path only)   */
  int32_t dtype;             /* TFM_DTYPE_*                              */
  int32_t route;             /* TFM_ROUTE_*                              */
  int32_t router;            /* TFM_ROUTER_*                             */
  float residual_multiplier; /* 1 for OLMoE; Granite's config value      */
} tfm_geometry;

typedef struct tfm_plan tfm_plan;

/* Validates the geometry and binds the plan to the current HIP device. */
int tfm_plan_create(const tfm_geometry* geometry, tfm_plan** plan_out);
void tfm_plan_destroy(tfm_plan* plan);

/* Bytes of workspace needed by calls on up to `tokens` tokens. */
size_t tfm_workspace_bytes(const tfm_plan* plan, int64_t tokens);

/* ---- weights --------------------------------------------------------- */
typedef struct tfm_affine {
  const uint32_t* q;  /* [E, N, Kin/8]     */
  const void* scales; /* [E, N, Kin/group] */
  const void* biases; /* [E, N, Kin/group] */
} tfm_affine;

typedef struct tfm_moe_weights {
  const void* router;       /* TFM_ROUTER_DENSE: router weight [E, H] in dtype */
  const float* logit_bias;  /* optional [E] fp32 added to the router logits
                               before rounding; no counterpart in the
                               reference (synthetic routing skew). NULL = none */
  tfm_affine gate, up, down;
  /* TFM_ROUTER_AFFINE: the router as an affine-quantised [E, H] matrix
   * (Q [E, H*router_bits/32], S/B [E, H/64] in dtype), the `mlp.gate` /
   * `router.layer` Affine of export_native_olmoe_target.py:160-171,194-200 and
   * export_native_granite_target.py:231-237. Logits are rounded to dtype. */
  tfm_affine router_affine;
  int32_t router_bits;      /* 4 or 8 (TFM_ROUTER_AFFINE only)             */
} tfm_moe_weights;

/* ---- routing --------------------------------------------------------- */
/* Router linear then routing. Replaces `linear(x, router)` + `route()`
 * (MLXNativeGraniteMoEPrefill.h:591-632; MLXOLMoERouter.h:86-120).
 *   x       [T, H] dtype
 *   logits  optional out [T, E] dtype (NULL = not returned)
 *   idx     out [T, K] int32, slot order of the reference
 *   gates   out [T, K]: dtype for OLMoE (probabilities), fp32 for Granite
 * Needs a TFM_ROUTER_DENSE plan with bf16 dtype. */
int tfm_route(const tfm_plan* plan, const void* x, int64_t tokens,
              const void* router, const float* logit_bias, void* logits,
              int32_t* idx, void* gates, void* workspace, size_t workspace_bytes,
              void* stream);

/* tfm_route for a TFM_ROUTER_AFFINE plan: the router linear is the
 * affine-quantised matmul of the exports' router module
 * (`torch.ops.mlx.native_affine_qmm(x, W, S, B, 64, bits)`,
 * export_native_olmoe_target.py:166-167,200; export_native_granite_target.py:236-237).
 * router: Q [E, H*router_bits/32], S/B [E, H/64] in dtype. Logits are
 * tree-reduced like the dense router's over w = dtype(s*q + b). */
int tfm_route_affine(const tfm_plan* plan, const void* x, int64_t tokens,
                     const tfm_affine* router, int32_t router_bits, const float* logit_bias,
                     void* logits, int32_t* idx, void* gates, void* workspace,
                     size_t workspace_bytes, void* stream);

/* Routing from given logits [T, E] (dtype). OLMoE: native_olmoe_softmax +
 * native_olmoe_topk_indices + native_take_along_last
 * (native_affine_ops.py:128-146); Granite: native_topk_indices +
 * take + fp32 softmax (export_native_granite_target.py:237-240). */
int tfm_route_logits(const tfm_plan* plan, const void* logits, int64_t tokens,
                     int32_t* idx, void* gates, void* stream);

/* OLMoE softmax only: probs [T, E] dtype (native_olmoe_softmax,
 * native_affine_ops.py:128-131). Needs E <= 64. */
int tfm_olmoe_softmax(const void* logits, int64_t tokens, int32_t num_experts,
                      int32_t dtype, void* probs, void* stream);

/* Top-k of given values [T, n] (dtype) without a softmax:
 *   rule TFM_ROUTE_OLMOE:   descending, ties to the lower index, NaN last
 *                           (native_olmoe_topk_indices, native_affine_ops.py:141-146;
 *                           MLXOLMoERouter.h:65-83)
 *   rule TFM_ROUTE_GRANITE: the k largest by a stable ascending rank (ties: higher
 *                           index selected), slots in ascending order
 *                           (native_topk_indices lowered as argpartition(-k) + slice,
 *                           native_affine_lowering.py:61-74; MLXNativeGraniteMoEPrefill.h:92-109)
 * idx out [T, k] int32. n <= 64. */
int tfm_topk(const void* values, int64_t tokens, int32_t n, int32_t k, int32_t rule,
             int32_t dtype, int32_t* idx, void* stream);

/* ---- grouping -------------------------------------------------------- */
/* Stable grouping of n flat routes by expert id
 * (MLXNativeGraniteMoEPrefill.h:666-684: argsort, inverse, take):
 *   order[pos] = flat index, sorted by (expert asc, flat asc)
 *   inverse[flat] = pos
 *   offsets[e] = first pos of expert e, offsets[E] = number of valid routes.
 * Ids outside [0,E) sort after every valid id and set
 * TFM_STATUS_BAD_EXPERT_ID in the workspace status word. */
size_t tfm_group_workspace_bytes(int64_t n_routes, int32_t num_experts);
int tfm_group(const int32_t* expert_ids, int64_t n_routes, int32_t num_experts,
              int32_t* order, int32_t* inverse, int32_t* offsets,
              void* workspace, size_t workspace_bytes, void* stream);

/* ---- gather_qmm ------------------------------------------------------ */
/* mlx::core::gather_qmm(x, w, scales, biases, nullopt, rhs_indices,
 * transpose=true, group, bits, "affine", sorted)
 * (MLXNativeGraniteMoEPrefill.h:542-550; op native_affine_gather_qmm,
 * native_affine_ops.py:55-63), flattened to rows:
 *   out[r, :] = x[x_rows[r], :] . W[rhs_indices[r]]^T      r in [0, rows)
 *   x [x_row_count, k_in] dtype; x_rows NULL means x_rows[r] = r (then
 *   x_row_count >= rows); out [rows, n_out] dtype. Out-of-range x_rows entries
 *   read row 0 and set TFM_STATUS_BAD_ROW_INDEX; out-of-range expert ids leave
 *   their rows unwritten and set TFM_STATUS_BAD_EXPERT_ID.
 * `sorted` is the caller's promise that rhs_indices is non-decreasing; results
 * do not depend on it. */
size_t tfm_gather_qmm_workspace_bytes(int64_t rows, int32_t num_experts,
                                      int32_t n_out, int32_t k_in);
int tfm_gather_qmm(const void* x, int64_t x_row_count, const int32_t* x_rows,
                   const int32_t* rhs_indices,
                   int64_t rows, const tfm_affine* w, int32_t num_experts,
                   int32_t n_out, int32_t k_in, int32_t group_size, int32_t bits,
                   int32_t dtype, int32_t sorted, void* out,
                   void* workspace, size_t workspace_bytes, void* stream);

/* ---- dense affine linear ---------------------------------------------- */
/* mlx::core::quantized_matmul(x, W, scales, biases, transpose=true, group,
 * bits, "affine") behind NativeLinearWeight::operator() (MLXNativeLinear.h:42-48;
 * op native_affine_qmm, native_affine_ops.py:39-52), flattened to rows:
 *   out[r, :] = x[r, :] . W^T      r in [0, rows)
 *   x [rows, k_in] dtype, w one matrix (Q [n_out, k_in*bits/32], S, B
 *   [n_out, k_in/group]), out [rows, n_out] dtype.
 * The same kernels as tfm_gather_qmm with one expert, without the grouping
 * pass and without a workspace. */
int tfm_affine_qmm(const void* x, int64_t rows, const tfm_affine* w, int32_t n_out,
                   int32_t k_in, int32_t group_size, int32_t bits, int32_t dtype, void* out,
                   void* stream);

/* ---- the MoE block --------------------------------------------------- */
/* Expert part of the block given routes: NativeMoEExpertHook::execute's
 * contract (MLXMoEExpertHook.h:43-51) - result = residual +
 * residual_multiplier * sum_k gates[t,k] * expert_{idx[t,k]}(x[t]),
 * in x's dtype. idx [T, K] int32, gates [T, K] fp32, residual optional
 * [T, H] (NULL = zeros), y out [T, H]. */
int tfm_moe_experts(const tfm_plan* plan, const void* x, int64_t tokens,
                    const void* residual, const int32_t* idx, const float* gates,
                    const tfm_moe_weights* weights, void* y, uint32_t flags,
                    void* workspace, size_t workspace_bytes, void* stream);

/* The whole block: tfm_route then tfm_moe_experts
 * (NativeGraniteMoEPrefill::moe, MLXNativeGraniteMoEPrefill.h:627-702).
 * idx_out [T,K] int32 and gates_out [T,K] fp32 are optional copies of the
 * routing (NULL = not returned). */
int tfm_moe_forward(const tfm_plan* plan, const void* x, int64_t tokens,
                    const void* residual, const tfm_moe_weights* weights, void* y,
                    int32_t* idx_out, float* gates_out, uint32_t flags,
                    void* workspace, size_t workspace_bytes, void* stream);

/* Allocation-free variant of tfm_moe_forward. No counterpart in the
 * reference: it is for callers that cannot allocate or pass device memory
 * (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc). Same arguments, kernels and results as tfm_moe_forward, but the
 * scratch memory is a static device array of TFM_STATIC_SCRATCH_BYTES inside
 * the library (one per GPU, held until the process ends) instead of a caller
 * workspace. Calls needing more scratch than that (tfm_workspace_bytes(plan,
 * tokens) > TFM_STATIC_SCRATCH_BYTES: past 776 tokens for OLMoE geometry
 * with a dense router, 773 with an affine one; past 1105 tokens for Granite
 * geometry, 1103 with an affine router) fail with TFM_E_WORKSPACE. The call allocates nothing. Every call on a GPU
 * shares that GPU's array: calls that overlap on one GPU (other streams,
 * other threads, other plans) race and must be ordered by the caller. Device
 * status bits (bad expert ids) of this variant are not reported. */
#define TFM_STATIC_SCRATCH_BYTES ((size_t)64 << 20)
int tfm_moe_forward_static(const tfm_plan* plan, const void* x, int64_t tokens,
                           const void* residual, const tfm_moe_weights* weights, void* y,
                           int32_t* idx_out, float* gates_out, uint32_t flags, void* stream);

/* The block with its neighbouring step fused in, as the reference layer runs
 * it (MLXNativeGraniteMoEPrefill.h:485-487):
 *   post = rms_norm(h, norm_weight, eps)          (fast::rms_norm, :485)
 *   y    = h + rm * sum_k gate_k * expert_k(post)   (moe(post, h, ...), :486, :688-701)
 * h, y: [T, H] in the plan dtype, y must not alias h; norm_weight: [H] in the
 * plan dtype. The RMSNorm order is bit-defined: lane l of 64 sums x*x over
 * its H/64 contiguous elements with sequential fma, a pairwise tree over
 * the lanes, mean = sum / H, inv = 1 / sqrt(mean + eps), then
 * post = round(w * round(h * inv)). Same workspace, outputs and flags as
 * tfm_moe_forward. */
int tfm_moe_forward_rmsnorm(const tfm_plan* plan, const void* h, int64_t tokens,
                            const void* norm_weight, float eps, const tfm_moe_weights* weights,
                            void* y, int32_t* idx_out, float* gates_out, uint32_t flags,
                            void* workspace, size_t workspace_bytes, void* stream);

/* NativeMoEExpertHook::GPUCallable (MLXMoEExpertHook.h:23-30,
 * MLXNativeGraniteMoEPrefill.h:635-658): for N parallel routes
 * (token_indices[i], expert_ids[i]) compute the expert outputs in expert-sorted
 * order, out_sorted [N, H] dtype, with inverse [N] int32 such that
 * out_sorted[inverse[i]] belongs to route i. experts_sorted != 0 is the
 * caller's promise that expert_ids is non-decreasing. N == 0 is allowed.
 * token_indices outside [0, tokens) read token 0 and set
 * TFM_STATUS_BAD_ROW_INDEX. */
size_t tfm_expert_routes_workspace_bytes(const tfm_plan* plan, int64_t n_routes);
int tfm_expert_routes(const tfm_plan* plan, const void* x, int64_t tokens,
                      const int32_t* token_indices, const int32_t* expert_ids,
                      int64_t n_routes, int32_t experts_sorted,
                      const tfm_moe_weights* weights, void* out_sorted,
                      int32_t* inverse, void* workspace, size_t workspace_bytes,
                      void* stream);

/* ---- stage profiler ---------------------------------------------------- */
/* Kernel stages of tfm_moe_forward / tfm_moe_experts. */
#define TFM_STAGE_ROUTER 0  /* router linear                               */
#define TFM_STAGE_TOPK 1    /* softmax + top-k                              */
#define TFM_STAGE_GROUP 2   /* stable grouping by expert                    */
#define TFM_STAGE_GATEUP 3  /* gate/up expert matmuls + SwiGLU              */
#define TFM_STAGE_DOWN 4    /* down expert matmul (+ gate weighting)        */
#define TFM_STAGE_COMBINE 5 /* K reduction + residual                       */
#define TFM_STAGE_NORM 6    /* post-attention RMSNorm (forward_rmsnorm)    */
#define TFM_STAGE_COUNT 7

/* Host-wall stage timing in the spirit of TriFuse's TRIFUSE_PREFILL_TIMING
 * stage lines (patches/executorch.patch:307-322), measured on the GPU: while
 * a profiler is attached to the calling thread, every stage of every MoE call
 * made on that thread is bracketed by two HIP events on the call's stream.
 * Up to `capacity` stage launches are recorded; later ones are counted as
 * dropped. tfm_profiler_stage waits for the recorded events and returns the
 * summed duration (ms) and the number of launches of one stage. */
typedef struct tfm_profiler tfm_profiler;
int tfm_profiler_create(int32_t capacity, tfm_profiler** out);
void tfm_profiler_destroy(tfm_profiler* profiler);
int tfm_profiler_attach(tfm_profiler* profiler); /* NULL detaches */
int tfm_profiler_reset(tfm_profiler* profiler);
int tfm_profiler_stage(tfm_profiler* profiler, int32_t stage, double* total_ms,
                       int32_t* launches, int32_t* dropped);
/* Kernel-exact duration of a stage: the main kernel of each recorded stage
 * launch (the first one it launches: the gate/up, down, combine, logits or
 * fused routing kernel) is launched with hipExtLaunchKernelGGL events, which
 * take the kernel dispatch's own start and end timestamps, the figures a
 * rocprofv3 kernel trace reports, without the launch and cache-release gaps
 * that the bracketing events of tfm_profiler_stage include. Returns the summed
 * kernel durations (ms) and how many stage launches had such a kernel. */
int tfm_profiler_stage_kernel(tfm_profiler* profiler, int32_t stage, double* kernel_ms,
                              int32_t* kernels);
const char* tfm_stage_name(int32_t stage);

/* ---- diagnostics ----------------------------------------------------- */
/* Blocking: synchronises `stream`, then reads and clears the device status
 * word kept in `workspace` (TFM_STATUS_* bits). The bits are sticky: a bad
 * expert id or row index seen by any call since the last read stays
 * reported, whatever later calls on the same workspace did. */
int tfm_status_word(void* workspace, void* stream, uint32_t* status_out);

/* Message of the last failing call on this thread ("" if none). */
const char* tfm_last_error(void);

/* Library version string. */
const char* tfm_version(void);

#ifdef __cplusplus
}
#endif
#endif /* TRIFUSE_MOE_H */
