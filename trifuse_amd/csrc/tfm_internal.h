// Internal host-side declarations shared by the library's translation units.
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include <string>
#include <utility>

#include "../../include/trifuse_moe.h"

namespace tfm {

// Status reporting: every entry point catches tfm::Error and returns its code.
struct Error {
  int code;
  std::string message;
};
[[noreturn]] void fail(int code, const std::string& message);
void check_hip(hipError_t err, const char* what);
void set_last_error(const std::string& message);

inline size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

// Kernel-exact stage timing. While a stage profiler is attached to the
// calling thread, each stage scope offers one event pair; the first kernel the
// stage launches through tfm_launch takes it with hipExtLaunchKernelGGL,
// which binds the events to the kernel dispatch itself (its start and end
// timestamps), so the pair measures the kernel alone.
struct KernelTimer {
  hipEvent_t start = nullptr, end = nullptr;
  bool used = false;
};
KernelTimer* pending_kernel_timer();  // the current stage's offer, or null

template <typename... P, typename... A>
inline void tfm_launch(void (*kernel)(P...), dim3 grid, dim3 block, size_t lds, hipStream_t s, A&&... args) {
  KernelTimer* t = pending_kernel_timer();
  if (t && !t->used) {
    t->used = true;
    hipExtLaunchKernelGGL(kernel, grid, block, (uint32_t)lds, s, t->start, t->end, 0u, std::forward<A>(args)...);
  } else {
    kernel<<<grid, block, lds, s>>>(std::forward<A>(args)...);
  }
}

// Workspace carve-up: regions are 256-byte aligned, in declaration order.
struct Carver {
  char* base;
  size_t offset = 0;
  explicit Carver(void* b) : base(static_cast<char*>(b)) {}
  template <typename T>
  T* take(size_t count) {
    offset = align_up(offset, 256);
    T* p = base ? reinterpret_cast<T*>(base + offset) : nullptr;
    offset += count * sizeof(T);
    return p;
  }
};

// Header at the start of every workspace.
struct WsHeader {
  uint32_t status;   // TFM_STATUS_* bits, sticky until tfm_status_word reads them
  uint32_t pad[63];
};
static_assert(sizeof(WsHeader) == 256, "workspace header size");

// Grouping results shared by every consumer of a route list.
struct Grouping {
  int32_t* order;    // [n] sorted position -> flat route
  int32_t* inverse;  // [n] flat route -> sorted position
  int32_t* offsets;  // [E+1]
  int32_t* active;   // [E+1] ids of experts with routes, ascending; active[E] = count
  int E;             // number of experts
  // Written by the decode gate/up kernel for the decode down GEMV (null on
  // other paths): per active slot s {expert, first route, end route, 0}
  // (slots past the active count hold expert -1), and the route gates in
  // sorted order.
  int4* slots;          // [E]
  float* gates_sorted;  // [n]
  // ident > 0: the identity grouping of a dense matrix (E == 1): expert 0
  // owns routes [0, ident) in caller order, and order, inverse, offsets and
  // active are not read (they may be null).
  int ident;
};

// Segment start of expert e (e <= E), the active-expert count and the id of
// active slot a, for both a written grouping and the identity one.
__device__ __forceinline__ int grp_offset(const Grouping& g, int e) {
  return g.ident ? (e == 0 ? 0 : g.ident) : g.offsets[e];
}
__device__ __forceinline__ int grp_active_count(const Grouping& g) { return g.ident ? 1 : g.active[g.E]; }
__device__ __forceinline__ int grp_active_id(const Grouping& g, int a) { return g.ident ? 0 : g.active[a]; }

// ---- launchers (defined in the .hip files) ----
void launch_router_logits(bool f16, const uint16_t* x, const uint16_t* w, const float* bias, int T,
                          int H, int E, uint16_t* logits, hipStream_t s);
// f16: logits/values/probabilities are IEEE half bits instead of bf16.
void launch_topk(int route_kind, bool f16, const uint16_t* logits, int T, int E, int K, int32_t* idx,
                 void* gates_native, float* gates_f32, hipStream_t s);
void launch_rank_topk(int rule, bool f16, const uint16_t* values, int T, int n, int K, int32_t* idx,
                      hipStream_t s);
void launch_olmoe_softmax(bool f16, const uint16_t* logits, int T, int E, uint16_t* probs, hipStream_t s);
// Affine-quantised router [E, H] (bits 4 or 8, group 64) dequantised into a
// dense [E, H] matrix w in the storage dtype, for the dense router kernels.
void launch_dequant_router(bool f16, int bits, const tfm_affine& r, int E, int H, uint16_t* w,
                           hipStream_t s);
// Grouping (group.hip): per-chunk expert histograms, then a stable scatter.
// hist holds group_blocks(n, chunk) rows of E+1 counts (bucket E: bad ids).
constexpr int kGroupChunk = 512;           // routes per chunk for given routes
constexpr int kTopkTokensPerBlock = 4;     // tokens per routing workgroup (chunk = 4*K)
int group_blocks(int64_t n, int chunk);
// Rows of E+1 counts the histogram workspace needs for nblocks chunks (the
// chunk histograms, then the superblock sums).
int group_hist_rows(int64_t nblocks);
void launch_group(const int32_t* ids, int64_t n, int E, Grouping g, int32_t* hist, uint32_t* status,
                  hipStream_t s);
// Scatter with chunk histograms already built (overwritten by chunk bases).
void launch_group_scatter(const int32_t* ids, int64_t n, int E, int chunk, int32_t* hist,
                          Grouping g, uint32_t* status, hipStream_t s);
// Top-k that also writes the chunk histograms (chunk = kTopkTokensPerBlock * K routes).
// Prefill routing in one kernel: logits (optionally written out), top-k and
// the chunk histogram of kTopkTokensPerBlock tokens per chunk. Returns false
// (nothing launched) for a hidden size it has no variant for.
bool launch_router_topk(int route_kind, bool f16, const uint16_t* x, const uint16_t* w, const float* bias,
                        int T, int H, int E, int K, int32_t* idx, float* gates_f32, int32_t* hist,
                        uint16_t* logits_out, hipStream_t s);
void launch_topk_hist(int route_kind, bool f16, const uint16_t* logits, int T, int E, int K, int32_t* idx,
                      float* gates_f32, int32_t* hist, hipStream_t s);

// Post-attention RMSNorm (norm.hip): out = st(w * st(x * inv)) in the storage
// dtype (bf16, or half when f16), one wave per row, bit-defined order.
void launch_rmsnorm(bool f16, const uint16_t* x, const uint16_t* w, float eps, int T, int H,
                    uint16_t* out, hipStream_t s);

// Decode path (decode.hip), T*K <= 256 routes.
// The decode logits on the affine router itself (bits 4 or 8), each row
// dequantised in the kernel as the dequant pass would round it; false (nothing
// launched) for a hidden size without a variant.
bool launch_decode_logits_affine(bool f16, int bits, const uint16_t* x, const tfm_affine& router, const float* bias,
                                 int T, int H, int E, uint16_t* logits, hipStream_t s);
void launch_decode_logits(bool f16, const uint16_t* x, const uint16_t* router, const float* bias, int T,
                          int H, int E, uint16_t* logits, hipStream_t s);

// Streaming decode path (dstream.hip). decode_stream_fits: the shapes it
// has variants for. ds_gateup routes (mode TFM_ROUTE_OLMOE/GRANITE: ranks
// logits [T,E] and writes idx/gates) or takes given routes (mode
// kDsGivenRoutes: reads idx/gates), groups them, publishes the grouping
// (g with g.slots and g.gates_sorted) and the status word, and writes the
// SwiGLU rows h in sorted order; ds_down reads the published grouping.
// Few tokens (decode_small): the down GEMV fused with the combine
// (y[t] = st(fma(rm, sum_k gate * out, residual)), rounded as the
// separate down GEMV and combine round it).
// One set per storage dtype and code width: ds_bf16 (dstream.hip), ds_f16
// (dstream_f16.hip), ds_bf16_i8 (dstream_i8.hip), ds_f16_i8 (dstream_f16_i8.hip).
constexpr int kDsGivenRoutes = 2;
// Small batches whose down projection runs fused with the combine
// (decode_small): at most kDsSmallT tokens and kDsSmallR routes.
constexpr int kDsSmallT = 3;
constexpr int kDsSmallR = 24;
// Row order of the gate/up kernel's h output: route order (h row f = flat
// route f) for one token with ranked routes whose down projection is the
// fused down + combine kernel (K <= kDsSmallR); expert-sorted order
// otherwise, which the separate down kernel reads.
__host__ __device__ inline bool ds_h_route_order(int mode, int T, int K) {
  return mode != kDsGivenRoutes && T == 1 && K <= kDsSmallR;
}
#define TFM_DS_DECLS                                                                                     \
  bool decode_stream_fits(int T, int K, int E, int H, int I);                                             \
  void launch_ds_gateup(int mode, const uint16_t* x, const uint16_t* logits, int32_t* idx, float* gates,  \
                        int T, int K, int E, int H, int I, const tfm_affine& gate, const tfm_affine& up,  \
                        const Grouping& g, uint32_t* status, uint16_t* h, const tfm_affine* pf_down,      \
                        hipStream_t s);                                                                   \
  void launch_ds_down(const uint16_t* hsorted, int H, int I, int max_active, const tfm_affine& down,      \
                      const Grouping& g, float* P, hipStream_t s);                                        \
  bool decode_small(int T, int K);                                                                        \
  void launch_ds_down_combine(const uint16_t* h, bool h_route_order, const int32_t* idx,                 \
                              const float* gates, const int32_t* inverse, int T, int K, int E, int H, int I, \
                              const tfm_affine& down, const uint16_t* residual, float rmul, uint16_t* y, \
                              hipStream_t s);                                                             \
  void launch_ds_route_group(int route_kind, const uint16_t* logits, int T, int E, int K, int32_t* idx,   \
                             float* gates, const Grouping& g, uint32_t* status, hipStream_t s);
namespace ds_bf16 { TFM_DS_DECLS }
namespace ds_f16 { TFM_DS_DECLS }
namespace ds_bf16_i8 { TFM_DS_DECLS }
namespace ds_f16_i8 { TFM_DS_DECLS }
#undef TFM_DS_DECLS
inline bool decode_stream_fits(int T, int K, int E, int H, int I) { return ds_bf16::decode_stream_fits(T, K, E, H, I); }
inline bool decode_small(int T, int K) { return ds_bf16::decode_small(T, K); }
// The build for storage dtype (f16: IEEE half, else bf16) and code width bits.
#define TFM_DS_PICK(f16, bits, call)      \
  do {                                    \
    if ((bits) == 8 && (f16))             \
      ds_f16_i8::call;                    \
    else if ((bits) == 8)                 \
      ds_bf16_i8::call;                   \
    else if (f16)                         \
      ds_f16::call;                       \
    else                                  \
      ds_bf16::call;                      \
  } while (0)
inline void launch_ds_gateup(bool f16, int bits, int mode, const uint16_t* x, const uint16_t* logits,
                             int32_t* idx, float* gates, int T, int K, int E, int H, int I,
                             const tfm_affine& gate, const tfm_affine& up, const Grouping& g,
                             uint32_t* status, uint16_t* h, hipStream_t s, const tfm_affine* pf_down = nullptr) {
  TFM_DS_PICK(f16, bits, launch_ds_gateup(mode, x, logits, idx, gates, T, K, E, H, I, gate, up, g, status, h, pf_down, s));
}
inline void launch_ds_down(bool f16, int bits, const uint16_t* hsorted, int H, int I, int max_active,
                           const tfm_affine& down, const Grouping& g, float* P, hipStream_t s) {
  TFM_DS_PICK(f16, bits, launch_ds_down(hsorted, H, I, max_active, down, g, P, s));
}
inline void launch_ds_down_combine(bool f16, int bits, const uint16_t* h, bool h_route_order,
                                   const int32_t* idx, const float* gates, const int32_t* inverse, int T,
                                   int K, int E, int H, int I, const tfm_affine& down,
                                   const uint16_t* residual, float rmul, uint16_t* y, hipStream_t s) {
  TFM_DS_PICK(f16, bits,
              launch_ds_down_combine(h, h_route_order, idx, gates, inverse, T, K, E, H, I, down, residual, rmul,
                                     y, s));
}
// Top-k and the stable grouping of at most 256 routes (T * K <= 256, E <= 64)
// in one workgroup, from logits [T, E] in the storage dtype: flat idx and fp32
// gates, then order, inverse, offsets, active list, slot table and sorted
// gates, and the status word, as the streaming gate/up kernel's prologue
// publishes them.
inline void launch_ds_route_group(bool f16, int route_kind, const uint16_t* logits, int T, int E, int K,
                                  int32_t* idx, float* gates, const Grouping& g, uint32_t* status, hipStream_t s) {
  if (f16)
    ds_f16::launch_ds_route_group(route_kind, logits, T, E, K, idx, gates, g, status, s);
  else
    ds_bf16::launch_ds_route_group(route_kind, logits, T, E, K, idx, gates, g, status, s);
}
#undef TFM_DS_PICK
// Also publishes the grouping (g, including g.slots and g.gates_sorted from
// the flat fp32 `gates`).
// Workgroups of decode_gateup_kernel's grid (row-unit blocks x active-slot
// bound) for a batch.
int decode_gateup_workgroups(int T, int K, int E, int H, int I);
void launch_decode_gateup(bool f16, const uint16_t* x, const int32_t* idx, const float* gates, int T, int E,
                          int K, int H, int I, const tfm_affine& gate, const tfm_affine& up,
                          const Grouping& g, uint16_t* h, uint32_t* status, hipStream_t s);

// Row source of a sorted route j: x row = x_rows ? x_rows[order[j]] : order[j] / K.
// Rows outside [0, nx) are read as row 0 and flag TFM_STATUS_BAD_ROW_INDEX.
// A null order is the identity (the dense matrix of an identity grouping).
struct RowMap {
  const int32_t* order;
  const int32_t* x_rows;  // may be null
  int K;                  // used when x_rows is null
  int64_t nx;             // rows of x
  uint32_t* status;       // workspace status word
};

__device__ __forceinline__ int route_flat(const RowMap& rm, int j) { return rm.order ? rm.order[j] : j; }

__device__ __forceinline__ int64_t route_row(const RowMap& rm, int j) {
  const int f = route_flat(rm, j);
  int64_t r = rm.x_rows ? (int64_t)rm.x_rows[f] : (int64_t)(f / rm.K);
  if (r < 0 || r >= rm.nx) {
    atomicOr(rm.status, (uint32_t)TFM_STATUS_BAD_ROW_INDEX);
    r = 0;
  }
  return r;
}

// Decode-style (few routes per expert) dequant GEMV family.
//   gateup: h[j, n] = st(silu(xg) * xu)              (sorted route j)
//   plain:  out[order[j], n] = st(x . w)              (gather_qmm)
//   scaled: P[j, n] = (x . w) * gate[order[j]]        (fp32, down + combine)
// st: the storage dtype (bf16, or IEEE half when f16); 4-bit codes.
// `routes` is the total route count (sizes the per-pass route batch).
void launch_gemv_gateup(bool f16, const uint16_t* x, RowMap rm, const Grouping& g, int max_active,
                        int64_t routes, const tfm_affine& gate, const tfm_affine& up, int N,
                        int Kin, uint16_t* h, hipStream_t s);
void launch_gemv_plain(bool f16, const uint16_t* x, RowMap rm, const Grouping& g, int max_active,
                       int64_t routes, const tfm_affine& w, int N, int Kin, uint16_t* out,
                       hipStream_t s);
void launch_gemv_scaled(bool f16, const uint16_t* hsorted, const Grouping& g, int max_active,
                        int64_t routes, const tfm_affine& w, int N, int Kin, const float* gates,
                        float* P, hipStream_t s);

// Grouped GEMM on expert-contiguous routes (prefill):
//   gateup: h[j, :] = bf16(silu(x W_gate^T) * (x W_up^T)) for sorted routes j
//   down:   y[j, :] = bf16(h[j, :] W_down^T)             (expert output, sorted j)
//   plain:  out[order[j], :] = bf16(x W^T)                 (gather_qmm)
void launch_ggemm_gateup(const uint16_t* x, RowMap rm, const Grouping& g, int64_t n_routes,
                         int E, const tfm_affine& gate, const tfm_affine& up, int N, int Kin,
                         int bits, bool f16, uint16_t* h, hipStream_t s);
void launch_ggemm_down(const uint16_t* hsorted, const Grouping& g, int64_t n_routes, int E,
                       const tfm_affine& w, int N, int Kin, int bits, bool f16, uint16_t* y_sorted,
                       hipStream_t s);
void launch_ggemm_plain(const uint16_t* x, RowMap rm, const Grouping& g, int64_t n_routes,
                        int E, const tfm_affine& w, int N, int Kin, int bits, bool f16, uint16_t* out,
                        hipStream_t s);

// Combine of gate-weighted fp32 rows (decode path):
//   y[t, c] = bf16(residual[t, c] + rm * sum_k P[inverse[t*K+k], c])   (k ascending)
// Routes whose sorted position is >= *n_valid (bad expert ids) contribute 0.
void launch_combine_sorted(bool f16, const float* P, const int32_t* inverse, const int32_t* n_valid, int T,
                           int K, int H, const uint16_t* residual, float rmul, uint16_t* y,
                           hipStream_t s);
// Combine of bf16 expert-output rows (prefill path):
//   y[t, c] = bf16(residual[t, c] + rm * sum_k gate[t*K+k] * Y[inverse[t*K+k], c])
// with the same k order and bad-route rule.
void launch_combine_rows(bool f16, const uint16_t* Y, const int32_t* inverse, const int32_t* n_valid,
                         const float* gates, int T, int K, int H, const uint16_t* residual,
                         float rmul, uint16_t* y, hipStream_t s);
// Expert-sorted output rows for the hook (decode path): out[j, c] = bf16(P[j, c])
void launch_rows_to_st(bool f16, const float* P, int64_t rows, int H, uint16_t* out, hipStream_t s);
void launch_copy_i32(const int32_t* src, int32_t* dst, int64_t n, hipStream_t s);

}  // namespace tfm
