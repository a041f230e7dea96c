// C ABI: plans, workspace layout, argument checks and launch orchestration.
//
// Orchestration follows NativeGraniteMoEPrefill::moe
// (MLXNativeGraniteMoEPrefill.h:627-702): router linear, route, grouping,
// up/gate expert matmuls with SwiGLU, down expert matmul, weighted combine and
// residual. The grouping is always the stable expert sort (the reference sorts
// once T*K >= 64; with fewer routes it gathers per route, which yields the
// same per-route results).
#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <string>
#include <vector>

#include "tfm_internal.h"

struct tfm_plan {
  tfm_geometry g;
  int device;
  int gemv_max_routes;  // route count up to which the decode GEMV path is used
  void* scratch;        // device address of this device's static scratch array (or null)
  std::string scratch_error;  // why `scratch` is null
};

// Stage profiler: HIP events recorded around each kernel stage of the calls
// made on a thread while the profiler is attached to it.
struct tfm_profiler {
  int capacity = 0;
  int used = 0;
  int dropped = 0;
  std::vector<hipEvent_t> start, end;
  std::vector<int> stage;
  std::vector<tfm::KernelTimer> kernel;  // per slot: the stage's main kernel, timed by its dispatch
};

namespace tfm {

// Workspace of the allocation-free entry point (tfm_moe_forward_static): a
// file-scope device array. Every GPU the library runs on holds its own copy
// until the process ends. In host code `scratch` is only a stand-in for the
// symbol: its device address (per device) comes from hipGetSymbolAddress,
// taken once per device in tfm_plan_create, and only that address is ever
// passed to kernels.
constexpr size_t kStaticScratchBytes = TFM_STATIC_SCRATCH_BYTES;
static __device__ __align__(256) uint8_t scratch[kStaticScratchBytes];
constexpr int kMaxDevices = 64;
static std::mutex g_scratch_mu;
static void* g_scratch_addr[kMaxDevices];

static thread_local std::string g_last_error;
static thread_local tfm_profiler* g_profiler = nullptr;
static thread_local KernelTimer* g_kernel_timer = nullptr;

KernelTimer* pending_kernel_timer() { return g_kernel_timer; }

// Records the stage's start event on construction and its end event on
// destruction when a profiler is attached to the calling thread, and offers
// the slot's kernel event pair to the first kernel the stage launches.
struct StageScope {
  tfm_profiler* p;
  int slot = -1;
  hipStream_t s;
  StageScope(int stage_id, hipStream_t stream) : p(g_profiler), s(stream) {
    if (!p) return;
    if (p->used >= p->capacity) {
      ++p->dropped;
      return;
    }
    slot = p->used++;
    p->stage[slot] = stage_id;
    p->kernel[slot].used = false;
    g_kernel_timer = &p->kernel[slot];
    (void)hipEventRecord(p->start[slot], s);
  }
  ~StageScope() {
    if (slot < 0) return;
    (void)hipEventRecord(p->end[slot], s);
    g_kernel_timer = nullptr;
  }
  StageScope(const StageScope&) = delete;
  StageScope& operator=(const StageScope&) = delete;
};

void set_last_error(const std::string& message) { g_last_error = message; }

[[noreturn]] void fail(int code, const std::string& message) { throw Error{code, message}; }

void check_hip(hipError_t err, const char* what) {
  if (err != hipSuccess) fail(TFM_E_HIP, std::string(what) + ": " + hipGetErrorString(err));
}

template <typename F>
static int guarded(F&& f) {
  try {
    f();
    g_last_error.clear();
    return TFM_OK;
  } catch (const Error& e) {
    g_last_error = e.message;
    return e.code;
  } catch (const std::exception& e) {
    g_last_error = std::string("internal error: ") + e.what();
    return TFM_E_INVALID;
  } catch (...) {
    g_last_error = "internal error";
    return TFM_E_INVALID;
  }
}

static void need(bool ok, const std::string& message) {
  if (!ok) fail(TFM_E_INVALID, message);
}

static void check_geometry(const tfm_geometry& g) {
  need(g.hidden_size > 0 && g.hidden_size % 64 == 0, "hidden_size must be a positive multiple of 64");
  need(g.intermediate_size > 0 && g.intermediate_size % 64 == 0,
       "intermediate_size must be a positive multiple of 64");
  need(g.num_experts > 0, "num_experts must be positive");
  need(g.experts_per_token > 0 && g.experts_per_token <= g.num_experts,
       "experts_per_token must be in [1, num_experts]");
  need(g.route == TFM_ROUTE_OLMOE || g.route == TFM_ROUTE_GRANITE, "unknown route kind");
  need(g.router == TFM_ROUTER_DENSE || g.router == TFM_ROUTER_AFFINE, "unknown router kind");
  need(g.dtype == TFM_DTYPE_BF16 || g.dtype == TFM_DTYPE_F16, "unknown dtype");
  need(g.bits == 4 || g.bits == 8, "bits must be 4 or 8");
  need(g.group_size == 32 || g.group_size == 64 || g.group_size == 128,
       "group_size must be 32, 64 or 128");
  if (g.num_experts > 64) fail(TFM_E_UNSUPPORTED, "num_experts > 64 is not built (wave-wide routing)");
  if (g.dtype == TFM_DTYPE_F16 && g.router != TFM_ROUTER_AFFINE)
    fail(TFM_E_UNSUPPORTED, "f16 blocks need the affine router (a dense f16 router is not built)");
  if (g.group_size != 64) fail(TFM_E_UNSUPPORTED, "only group_size 64 is built");
}

// Workspace of the MoE block for T tokens. base == nullptr computes sizes.
struct BlockWs {
  WsHeader* hdr;
  uint16_t* logits;
  int32_t* idx;
  float* gates;
  Grouping grp;
  uint16_t* h;
  float* P;  // [R, H] sorted rows (fp32 in decode, bf16 expert outputs in prefill)
  int32_t* hist;  // grouping chunk histograms
  int4* slots;    // decode: per active slot {expert, first route, end route, 0}
  float* gates_sorted;  // decode: gates in sorted order
  uint16_t* xn;         // RMSNorm-ed input [T, H] (tfm_moe_forward_rmsnorm)
  uint16_t* router_w;   // affine router dequantised to [E, H] (TFM_ROUTER_AFFINE)
  size_t bytes;
};

static BlockWs carve_block(const tfm_geometry& g, int64_t T, void* base) {
  const int64_t R = T * g.experts_per_token;
  Carver c(base);
  BlockWs w{};
  w.hdr = c.take<WsHeader>(1);
  w.logits = c.take<uint16_t>((size_t)(T * g.num_experts));
  w.idx = c.take<int32_t>((size_t)R);
  w.gates = c.take<float>((size_t)R);
  w.grp.order = c.take<int32_t>((size_t)R);
  w.grp.inverse = c.take<int32_t>((size_t)R);
  w.grp.offsets = c.take<int32_t>((size_t)g.num_experts + 1);
  w.grp.active = c.take<int32_t>((size_t)g.num_experts + 1);
  w.grp.E = g.num_experts;
  w.h = c.take<uint16_t>((size_t)(R * g.intermediate_size));
  w.P = c.take<float>((size_t)(R * g.hidden_size));
  const int64_t chunks = std::max<int64_t>(group_blocks(R, kGroupChunk),
                                           group_blocks(R, kTopkTokensPerBlock * g.experts_per_token));
  w.hist = c.take<int32_t>((size_t)group_hist_rows(chunks) * (g.num_experts + 1));
  w.slots = c.take<int4>((size_t)g.num_experts);
  w.gates_sorted = c.take<float>((size_t)R);
  w.xn = c.take<uint16_t>((size_t)(T * g.hidden_size));
  if (g.router == TFM_ROUTER_AFFINE)
    w.router_w = c.take<uint16_t>((size_t)g.num_experts * (size_t)g.hidden_size);
  w.bytes = align_up(c.offset, 256);
  return w;
}

// The decode path (routing per token, grouping in the gate/up prologue)
// applies when every route fits one grouping thread and both matmul widths
// fit one 32-element chunk per lane.
// The streaming decode kernels read 4-bit or 8-bit weights in bf16 or half
// storage (an affine router is dequantised first).
// Batches past the streaming decode kernels run the decode GEMV kernels
// rather than the grouped GEMM (64-row tiles) up to gemv_threshold() routes.

// Tokens up to which the streaming decode kernels take a batch that the
// decode GEMV kernels (4-bit codes, bf16 or half storage) could also run;
// past it the GEMV kernels do (TFM_DS_MAX_TOKENS overrides; an affine router
// is dequantised first on either path). Batches no GEMV kernel runs (8-bit
// codes) stream whenever they fit.
// Per layer, streaming against GEMV: OLMoE 1 token 16.8 against 22.4 us,
// 2 tokens 26.4 against 29.6, 3 tokens 35.5 against 34.6, 8 tokens (16
// layers) 56.0 against 53.0, 12 tokens 75.6 against 63.2; Granite 1 token
// 12.6 against 18.0, 2 tokens 17.6 against 21.1, 3 tokens 23.9 against 23.9,
// 8 tokens 34.9 against 32.5. The streaming layer of 1 to 3 tokens is three
// kernels (the down projection fused with the combine): 3 tokens went from
// 35.3 to 32.2 us (OLMoE) and from 24.4 to 21.6 (Granite) with it, against
// 34.6 and 23.9 on the GEMV kernels.
static int ds_max_tokens() {
  static const int v = [] {
    const char* s = std::getenv("TFM_DS_MAX_TOKENS");
    if (!s) return 3;
    char* end = nullptr;
    const long n = std::strtol(s, &end, 10);
    if (!end || end == s || *end != 0 || n < 0 || n > 256) {
      std::fprintf(stderr, "trifuse_moe: ignoring invalid TFM_DS_MAX_TOKENS=%s\n", s);
      return 3;
    }
    return (int)n;
  }();
  return v;
}

// Grouping of the decode GEMV path (TFM_DECODE_GROUPING=slots|workgroup
// forces one). With many gate/up workgroups (at least 4096: OLMoE from 4
// tokens), one route-and-group workgroup publishes the slot table after the
// logits and every gate/up workgroup reads its slot (gemv_kernel); with few
// (Granite), the multi-workgroup top-k runs instead and every gate/up
// workgroup groups the routes itself (decode_gateup_kernel). Reading a slot
// instead of grouping shortens each gate/up workgroup's prologue (1.7 us of
// route-id read and grouping at batch 8), which pays off only over many
// workgroups. Per layer, slots against in-workgroup grouping, one box:
// OLMoE 4 tokens 39.3 against 39.4 us, 8 tokens (16 layers) 53.6 against
// 55.5, 12 tokens 64.1 against 65.4; Granite 4 tokens 27.8 against 26.3,
// 8 tokens 34.2 against 33.2.
static bool decode_slot_grouping(int T, int K, int E, int H, int I) {
  static const int o = [] {
    const char* s = std::getenv("TFM_DECODE_GROUPING");
    if (!s) return -1;
    if (!std::strcmp(s, "slots")) return 1;
    if (!std::strcmp(s, "workgroup")) return 0;
    std::fprintf(stderr, "trifuse_moe: ignoring invalid TFM_DECODE_GROUPING=%s\n", s);
    return -1;
  }();
  if (o >= 0) return o == 1;
  return decode_gateup_workgroups(T, K, E, H, I) >= 4096;
}

// Whether the gate/up kernel of 1 to 3 tokens also copies the routed
// experts' down weights toward the down + combine kernel (TFM_DS_PREFETCH=1;
// off by default). Off measured faster once both kernels issued their loads
// early: per layer on one box, with against without, OLMoE 1 token 16.94
// against 16.83 us, 2 tokens 26.9 against 24.9; Granite 1 token 12.87
// against 12.39.
static bool ds_prefetch() {
  static const bool v = [] {
    const char* s = std::getenv("TFM_DS_PREFETCH");
    return s != nullptr && std::strcmp(s, "1") == 0;
  }();
  return v;
}

// Tokens up to which the prefill-path routing runs as two kernels (router
// logits with one wave per few (token, expert) pairs, then top-k with the
// chunk histograms) rather than the fused router + top-k kernel, whose
// 4-token workgroups leave most of the chip idle on small batches. Per
// layer, fused against split: OLMoE 32 tokens 120.0 against 112.0 us,
// 128 tokens 174.5 against 168.5, 512 tokens 141.4 against 139.6, 1024
// tokens 205.9 against 207.5, 4096 tokens (Zipf) 527.6 against 532.0;
// Granite decode 32 41.6 against 38.1. TFM_ROUTER_SPLIT_MAX_TOKENS overrides.
static int router_split_max_tokens() {
  static const int v = [] {
    const char* s = std::getenv("TFM_ROUTER_SPLIT_MAX_TOKENS");
    if (!s) return 512;
    char* end = nullptr;
    const long n = std::strtol(s, &end, 10);
    if (!end || end == s || *end != 0 || n < 0 || n > (1 << 30)) {
      std::fprintf(stderr, "trifuse_moe: ignoring invalid TFM_ROUTER_SPLIT_MAX_TOKENS=%s\n", s);
      return 512;
    }
    return (int)n;
  }();
  return v;
}

static bool fused_decode(const tfm_geometry& g, int64_t R) {
  return R <= 256 && g.hidden_size <= 2048 && g.intermediate_size <= 2048;
}

// Decode path override for measurement, read once (TFM_DECODE_PATH): 1
// streaming kernels (where they fit), 2 decode GEMV kernels (4-bit codes,
// whatever the route count), 3 grouped GEMM; 0 (unset) the automatic choice.
static int decode_path_override() {
  static const int v = [] {
    const char* s = std::getenv("TFM_DECODE_PATH");
    if (!s) return 0;
    if (!std::strcmp(s, "stream")) return 1;
    if (!std::strcmp(s, "gemv")) return 2;
    if (!std::strcmp(s, "gemm")) return 3;
    std::fprintf(stderr, "trifuse_moe: ignoring invalid TFM_DECODE_PATH=%s\n", s);
    return 0;
  }();
  return v;
}

// The decode path of a block: streaming kernels, decode GEMV kernels or (both
// false) the grouped GEMM.
struct DecodeChoice {
  bool stream, gemv;
};
static DecodeChoice decode_choice(const tfm_geometry& g, int64_t R, int gemv_max_routes) {
  const int T = (int)(R / g.experts_per_token);
  const bool fused = fused_decode(g, R);
  const bool fits = fused && decode_stream_fits(T, g.experts_per_token, g.num_experts, g.hidden_size,
                                                g.intermediate_size);
  const bool gemv_ok = fused && g.bits == 4;  // the GEMV kernels take 4-bit codes
  switch (decode_path_override()) {
    case 1: if (fits) return {true, false}; break;
    case 2: if (gemv_ok) return {false, true}; break;
    case 3: return {false, false};
    default: break;
  }
  // 4-bit codes: streaming kernels up to ds_max_tokens(), then the GEMV
  // kernels, then the grouped GEMM (faster than the streaming kernels there:
  // OLMoE 14 tokens 70.5 against 83.6 us, Granite 16 tokens 37.2 against
  // 50.7). 8-bit codes, which no GEMV kernel runs: streaming wherever the
  // token rows fit (8 tokens: 84 against 140 us on the grouped GEMM).
  const bool stream_small = fits && T <= ds_max_tokens();
  const bool gemv = gemv_ok && !stream_small && R <= gemv_max_routes;
  return {stream_small || (fits && !gemv_ok), gemv};
}


struct GroupWs {
  WsHeader* hdr;
  Grouping grp;
  int32_t* hist;
  size_t bytes;
};

static GroupWs carve_group(int64_t n, int E, void* base) {
  Carver c(base);
  GroupWs w{};
  w.hdr = c.take<WsHeader>(1);
  w.grp.order = c.take<int32_t>((size_t)n);
  w.grp.inverse = c.take<int32_t>((size_t)n);
  w.grp.offsets = c.take<int32_t>((size_t)E + 1);
  w.grp.active = c.take<int32_t>((size_t)E + 1);
  w.grp.E = E;
  w.hist = c.take<int32_t>((size_t)group_hist_rows(group_blocks(n, kGroupChunk)) * (E + 1));
  w.bytes = align_up(c.offset, 256);
  return w;
}

static void need_ws(void* ws, size_t have, size_t want) {
  if (!ws) fail(TFM_E_WORKSPACE, "workspace is null");
  if ((reinterpret_cast<uintptr_t>(ws) & 255) != 0) fail(TFM_E_WORKSPACE, "workspace must be 256-byte aligned");
  if (have < want)
    fail(TFM_E_WORKSPACE, "workspace too small: " + std::to_string(have) + " < " + std::to_string(want));
}

static void need_ptr(const void* p, const char* name) {
  if (!p) fail(TFM_E_INVALID, std::string(name) + " is null");
}

static void need_align16(const void* p, const char* name) {
  if (reinterpret_cast<uintptr_t>(p) & 15) fail(TFM_E_INVALID, std::string(name) + " must be 16-byte aligned");
}

static void check_affine(const tfm_affine& a, const char* name) {
  need_ptr(a.q, name);
  need_ptr(a.scales, name);
  need_ptr(a.biases, name);
  need_align16(a.q, name);
}

// Routes up to which expert products run the GEMV kernels (decode.hip,
// gemv.hip) instead of the grouped GEMM. TFM_GEMV_MAX_ROUTES (an integer in
// [0, 2^30]) sets it for every entry point; -1 when unset.
static int gemv_threshold_env() {
  static int v = [] {
    const char* s = std::getenv("TFM_GEMV_MAX_ROUTES");
    if (!s) return -1;
    char* end = nullptr;
    const long n = std::strtol(s, &end, 10);
    if (!end || end == s || *end != 0 || n < 0 || n > (1 << 30)) {
      std::fprintf(stderr, "trifuse_moe: ignoring invalid TFM_GEMV_MAX_ROUTES=%s\n", s);
      return -1;
    }
    return (int)n;
  }();
  return v;
}

// tfm_gather_qmm and tfm_affine_qmm without a plan: 176 routes.
static int gemv_threshold() {
  const int v = gemv_threshold_env();
  return v >= 0 ? v : 176;
}

// The MoE block (forward, hook and GPUCallable paths alike, so that they run
// the same kernels on the same routes): E + 40 routes, at most 176. Since the
// grouped GEMM's four-wave 64-row tiles the GEMM wins from a little under two
// routes per expert. Per layer, decode GEMV against grouped GEMM: OLMoE 12
// tokens (96 routes) 63.8 against 69.2 us, 13 tokens 67.5 against 70.2, 14
// tokens 70.7 against 70.5, 16 tokens 74.6 against 71.5, 20 tokens 82.9
// against 73.1; Granite 10 tokens (80 routes) 36.1 against 36.8, 11 tokens
// 37.6 against 36.9, 16 tokens 43.7 against 37.2, 20 tokens 49.7 against
// 38.0, decode 32 63.3 against 39.2.
static int block_gemv_threshold(int E) {
  const int v = gemv_threshold_env();
  return v >= 0 ? v : std::min(176, E + 40);
}

// Expert part of the block on grouped routes (flat routes t*K+k of idx).
// `grouped`: the routes in ws.grp already come grouped (prefill forward path).
static void run_experts(const tfm_plan* p, const uint16_t* x, int64_t T, const uint16_t* residual,
                        const int32_t* idx, const float* gates, const tfm_moe_weights* w,
                        uint16_t* y, uint32_t flags, BlockWs& ws, hipStream_t s,
                        bool grouped = false) {
  const tfm_geometry& g = p->g;
  const int H = g.hidden_size, I = g.intermediate_size, E = g.num_experts, K = g.experts_per_token;
  const int64_t R = T * K;
  const bool f16 = g.dtype == TFM_DTYPE_F16;
  // The path tfm_moe_forward takes for these routes, so that both entry
  // points run the same kernels (the GEMV kernels take 4-bit codes, bf16 or
  // half storage).
  const DecodeChoice dc = decode_choice(g, R, p->gemv_max_routes);
  const bool gemv = dc.gemv && H <= 2048 && I <= 2048;
  if (!grouped && dc.stream) {
    // Streaming decode kernels, the same ones tfm_moe_forward runs at decode
    // shapes, so both entry points give bit-identical results.
    Grouping gd = ws.grp;
    gd.slots = ws.slots;
    gd.gates_sorted = ws.gates_sorted;
    {
      StageScope st(TFM_STAGE_GATEUP, s);
      launch_ds_gateup(f16, g.bits, kDsGivenRoutes, x, nullptr, const_cast<int32_t*>(idx), const_cast<float*>(gates),
                       (int)T, K, E, H, I, w->gate, w->up, gd, &ws.hdr->status, ws.h, s,
                       ds_prefetch() ? &w->down : nullptr);
    }
    if (decode_small((int)T, K)) {
      StageScope st(TFM_STAGE_DOWN, s);
      launch_ds_down_combine(f16, g.bits, ws.h, ds_h_route_order(kDsGivenRoutes, (int)T, K), idx, gates,
                             ws.grp.inverse, (int)T, K, E, H, I, w->down, residual, g.residual_multiplier, y, s);
      return;
    }
    const int max_active = (int)(R < E ? R : E);
    {
      StageScope st(TFM_STAGE_DOWN, s);
      launch_ds_down(f16, g.bits, ws.h, H, I, max_active, w->down, gd, ws.P, s);
    }
    StageScope st(TFM_STAGE_COMBINE, s);
    launch_combine_sorted(f16, ws.P, ws.grp.inverse, ws.grp.offsets + E, (int)T, K, H, residual,
                          g.residual_multiplier, y, s);
    return;
  }
  if (!grouped) {
    StageScope st(TFM_STAGE_GROUP, s);
    launch_group(idx, R, E, ws.grp, ws.hist, &ws.hdr->status, s);
  }
  const int max_active = (int)(R < E ? R : E);
  const RowMap rm{ws.grp.order, nullptr, K, T, &ws.hdr->status};
  if (gemv) {
    {
      StageScope st(TFM_STAGE_GATEUP, s);
      launch_gemv_gateup(f16, x, rm, ws.grp, max_active, R, w->gate, w->up, I, H, ws.h, s);
    }
    {
      StageScope st(TFM_STAGE_DOWN, s);
      launch_gemv_scaled(f16, ws.h, ws.grp, max_active, R, w->down, H, I, gates, ws.P, s);
    }
    StageScope st(TFM_STAGE_COMBINE, s);
    launch_combine_sorted(f16, ws.P, ws.grp.inverse, ws.grp.offsets + E, (int)T, K, H, residual,
                          g.residual_multiplier, y, s);
  } else {
    // Prefill: the down projection writes bf16 expert outputs in sorted
    // order (into the P region), the combine weights and sums them per token.
    (void)flags;
    uint16_t* Y = reinterpret_cast<uint16_t*>(ws.P);
    {
      StageScope st(TFM_STAGE_GATEUP, s);
      launch_ggemm_gateup(x, rm, ws.grp, R, E, w->gate, w->up, I, H, g.bits, f16, ws.h, s);
    }
    {
      StageScope st(TFM_STAGE_DOWN, s);
      launch_ggemm_down(ws.h, ws.grp, R, E, w->down, H, I, g.bits, f16, Y, s);
    }
    StageScope st(TFM_STAGE_COMBINE, s);
    launch_combine_rows(f16, Y, ws.grp.inverse, ws.grp.offsets + E, gates, (int)T, K, H, residual,
                        g.residual_multiplier, y, s);
  }
}

// Device address of the static scratch array on `dev` (the current device),
// looked up once per device. A failed lookup is recorded in `why` and leaves
// nullptr: plans still work through the workspace entry points, and
// tfm_moe_forward_static reports the failure.
static void* static_scratch(int dev, std::string& why) {
  if (dev < 0 || dev >= kMaxDevices) {
    why = "device ordinal beyond the static scratch table";
    return nullptr;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_addr[dev]) {
    void* ptr = nullptr;
    const hipError_t err = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (err != hipSuccess || !ptr) {
      (void)hipGetLastError();
      why = std::string("hipGetSymbolAddress: ") + hipGetErrorString(err);
      return nullptr;
    }
    g_scratch_addr[dev] = ptr;
  }
  return g_scratch_addr[dev];
}

static void check_weights(const tfm_moe_weights* w, bool router, const tfm_geometry& g) {
  need_ptr(w, "weights");
  if (router && g.router == TFM_ROUTER_DENSE) {
    need_ptr(w->router, "weights->router");
    need_align16(w->router, "weights->router");
  } else if (router) {
    need(w->router_bits == 4 || w->router_bits == 8, "weights->router_bits must be 4 or 8");
    check_affine(w->router_affine, "weights->router_affine");
  }
  check_affine(w->gate, "weights->gate");
  check_affine(w->up, "weights->up");
  check_affine(w->down, "weights->down");
}

}  // namespace tfm

using namespace tfm;

extern "C" {

const char* tfm_last_error(void) { return g_last_error.c_str(); }

const char* tfm_version(void) { return "trifuse_moe 0.1 gfx950"; }

int tfm_plan_create(const tfm_geometry* geometry, tfm_plan** plan_out) {
  return guarded([&] {
    need_ptr(geometry, "geometry");
    need_ptr(plan_out, "plan_out");
    *plan_out = nullptr;
    check_geometry(*geometry);
    int dev = 0;
    check_hip(hipGetDevice(&dev), "hipGetDevice");
    std::string why;
    void* scr = static_scratch(dev, why);
    tfm_plan* p = new tfm_plan{};
    p->g = *geometry;
    p->device = dev;
    p->gemv_max_routes = block_gemv_threshold(geometry->num_experts);
    p->scratch = scr;
    p->scratch_error = why;
    *plan_out = p;
  });
}

void tfm_plan_destroy(tfm_plan* plan) { delete plan; }

size_t tfm_workspace_bytes(const tfm_plan* plan, int64_t tokens) {
  if (!plan || tokens < 0) return 0;
  return carve_block(plan->g, tokens, nullptr).bytes;
}

size_t tfm_group_workspace_bytes(int64_t n_routes, int32_t num_experts) {
  if (n_routes < 0 || num_experts <= 0) return 0;
  return carve_group(n_routes, num_experts, nullptr).bytes;
}

int tfm_route(const tfm_plan* plan, const void* x, int64_t tokens, const void* router,
              const float* logit_bias, void* logits, int32_t* idx, void* gates, void* workspace,
              size_t workspace_bytes, void* stream) {
  return guarded([&] {
    need_ptr(plan, "plan");
    need(tokens >= 0 && tokens <= INT32_MAX / 64, "tokens out of range");
    if (tokens == 0) return;
    need_ptr(x, "x");
    need_ptr(router, "router");
    need_ptr(idx, "idx");
    need_align16(x, "x");
    need_align16(router, "router");
    const tfm_geometry& g = plan->g;
    if (g.router != TFM_ROUTER_DENSE || g.dtype != TFM_DTYPE_BF16)
      fail(TFM_E_UNSUPPORTED, "tfm_route needs a dense-router bf16 plan (use tfm_route_affine)");
    BlockWs ws = carve_block(g, tokens, workspace);
    need_ws(workspace, workspace_bytes, ws.bytes);
    hipStream_t s = static_cast<hipStream_t>(stream);
    uint16_t* lg = logits ? static_cast<uint16_t*>(logits) : ws.logits;
    launch_router_logits(false, static_cast<const uint16_t*>(x), static_cast<const uint16_t*>(router),
                         logit_bias, (int)tokens, g.hidden_size, g.num_experts, lg, s);
    launch_topk(g.route, false, lg, (int)tokens, g.num_experts, g.experts_per_token, idx, gates,
                nullptr, s);
  });
}

int tfm_route_affine(const tfm_plan* plan, const void* x, int64_t tokens, const tfm_affine* router,
                     int32_t router_bits, const float* logit_bias, void* logits, int32_t* idx,
                     void* gates, void* workspace, size_t workspace_bytes, void* stream) {
  return guarded([&] {
    need_ptr(plan, "plan");
    need(tokens >= 0 && tokens <= INT32_MAX / 64, "tokens out of range");
    const tfm_geometry& g = plan->g;
    if (g.router != TFM_ROUTER_AFFINE) fail(TFM_E_INVALID, "tfm_route_affine needs an affine-router plan");
    need(router_bits == 4 || router_bits == 8, "router_bits must be 4 or 8");
    if (tokens == 0) return;
    need_ptr(x, "x");
    need_ptr(router, "router");
    need_ptr(idx, "idx");
    need_align16(x, "x");
    check_affine(*router, "router");
    BlockWs ws = carve_block(g, tokens, workspace);
    need_ws(workspace, workspace_bytes, ws.bytes);
    hipStream_t s = static_cast<hipStream_t>(stream);
    const bool f16 = g.dtype == TFM_DTYPE_F16;
    uint16_t* lg = logits ? static_cast<uint16_t*>(logits) : ws.logits;
    launch_dequant_router(f16, router_bits, *router, g.num_experts, g.hidden_size, ws.router_w, s);
    launch_router_logits(f16, static_cast<const uint16_t*>(x), ws.router_w, logit_bias, (int)tokens,
                         g.hidden_size, g.num_experts, lg, s);
    launch_topk(g.route, f16, lg, (int)tokens, g.num_experts, g.experts_per_token, idx, gates, nullptr, s);
  });
}

int tfm_route_logits(const tfm_plan* plan, const void* logits, int64_t tokens, int32_t* idx,
                     void* gates, void* stream) {
  return guarded([&] {
    need_ptr(plan, "plan");
    need(tokens >= 0 && tokens <= INT32_MAX / 64, "tokens out of range");
    if (tokens == 0) return;
    need_ptr(logits, "logits");
    need_ptr(idx, "idx");
    const tfm_geometry& g = plan->g;
    launch_topk(g.route, g.dtype == TFM_DTYPE_F16, static_cast<const uint16_t*>(logits), (int)tokens, g.num_experts,
                g.experts_per_token, idx, gates, nullptr, static_cast<hipStream_t>(stream));
  });
}

int tfm_topk(const void* values, int64_t tokens, int32_t n, int32_t k, int32_t rule,
             int32_t dtype, int32_t* idx, void* stream) {
  return guarded([&] {
    need(tokens >= 0 && tokens <= INT32_MAX / 64, "tokens out of range");
    need(n > 0 && k > 0 && k <= n, "need 0 < k <= n");
    need(rule == TFM_ROUTE_OLMOE || rule == TFM_ROUTE_GRANITE, "unknown top-k rule");
    if (n > 64) fail(TFM_E_UNSUPPORTED, "top-k over more than 64 values is not built");
    need(dtype == TFM_DTYPE_BF16 || dtype == TFM_DTYPE_F16, "unknown dtype");
    if (tokens == 0) return;
    need_ptr(values, "values");
    need_ptr(idx, "idx");
    launch_rank_topk(rule, dtype == TFM_DTYPE_F16, static_cast<const uint16_t*>(values), (int)tokens, n, k, idx,
                     static_cast<hipStream_t>(stream));
  });
}

int tfm_olmoe_softmax(const void* logits, int64_t tokens, int32_t num_experts, int32_t dtype,
                      void* probs, void* stream) {
  return guarded([&] {
    need(tokens >= 0 && tokens <= INT32_MAX / 64, "tokens out of range");
    need(num_experts > 0, "num_experts must be positive");
    if (num_experts > 64) fail(TFM_E_UNSUPPORTED, "num_experts > 64 is not built");
    need(dtype == TFM_DTYPE_BF16 || dtype == TFM_DTYPE_F16, "unknown dtype");
    if (tokens == 0) return;
    need_ptr(logits, "logits");
    need_ptr(probs, "probs");
    launch_olmoe_softmax(dtype == TFM_DTYPE_F16, static_cast<const uint16_t*>(logits), (int)tokens, num_experts,
                         static_cast<uint16_t*>(probs), static_cast<hipStream_t>(stream));
  });
}

int tfm_group(const int32_t* expert_ids, int64_t n_routes, int32_t num_experts, int32_t* order,
              int32_t* inverse, int32_t* offsets, void* workspace, size_t workspace_bytes,
              void* stream) {
  return guarded([&] {
    need(n_routes >= 0 && n_routes <= INT32_MAX, "n_routes out of range");
    need(num_experts > 0, "num_experts must be positive");
    if (num_experts > 64) fail(TFM_E_UNSUPPORTED, "num_experts > 64 is not built");
    need_ptr(offsets, "offsets");
    GroupWs ws = carve_group(n_routes, num_experts, workspace);
    need_ws(workspace, workspace_bytes, ws.bytes);
    if (n_routes > 0) {
      need_ptr(expert_ids, "expert_ids");
      need_ptr(order, "order");
      need_ptr(inverse, "inverse");
    }
    Grouping gout = ws.grp;
    gout.order = order;
    gout.inverse = inverse;
    gout.offsets = offsets;
    launch_group(expert_ids, n_routes, num_experts, gout, ws.hist, &ws.hdr->status,
                 static_cast<hipStream_t>(stream));
  });
}

size_t tfm_gather_qmm_workspace_bytes(int64_t rows, int32_t num_experts, int32_t n_out,
                                      int32_t k_in) {
  (void)n_out;
  (void)k_in;
  if (rows < 0 || num_experts <= 0) return 0;
  return carve_group(rows, num_experts, nullptr).bytes;
}

int tfm_gather_qmm(const void* x, int64_t x_row_count, const int32_t* x_rows,
                   const int32_t* rhs_indices, int64_t rows,
                   const tfm_affine* w, int32_t num_experts, int32_t n_out, int32_t k_in,
                   int32_t group_size, int32_t bits, int32_t dtype, int32_t sorted, void* out,
                   void* workspace, size_t workspace_bytes, void* stream) {
  (void)sorted;
  return guarded([&] {
    need(rows >= 0 && rows <= INT32_MAX, "rows out of range");
    need(x_row_count >= 0, "x_row_count out of range");
    need(x_rows || x_row_count >= rows, "x_row_count < rows with identity x_rows");
    need(num_experts > 0, "num_experts must be positive");
    need(n_out > 0 && k_in > 0, "n_out and k_in must be positive");
    need(bits == 4 || bits == 8, "bits must be 4 or 8");
    need(group_size == 32 || group_size == 64 || group_size == 128, "group_size must be 32, 64 or 128");
    need(k_in % group_size == 0, "k_in must be a multiple of group_size");
    if (num_experts > 64) fail(TFM_E_UNSUPPORTED, "num_experts > 64 is not built");
    if (group_size != 64) fail(TFM_E_UNSUPPORTED, "only group_size 64 is built");
    need(dtype == TFM_DTYPE_BF16 || dtype == TFM_DTYPE_F16, "unknown dtype");
    if (n_out % 64 != 0) fail(TFM_E_UNSUPPORTED, "n_out must be a multiple of 64");
    GroupWs ws = carve_group(rows, num_experts, workspace);
    need_ws(workspace, workspace_bytes, ws.bytes);
    if (rows == 0) return;
    need(x_row_count > 0, "x has no rows to gather from");
    need_ptr(x, "x");
    need_ptr(rhs_indices, "rhs_indices");
    need_ptr(w, "w");
    need_ptr(out, "out");
    need_align16(x, "x");
    check_affine(*w, "w");
    hipStream_t s = static_cast<hipStream_t>(stream);
    launch_group(rhs_indices, rows, num_experts, ws.grp, ws.hist, &ws.hdr->status, s);
    // x_rows == nullptr means identity: RowMap uses f / K with K = 1.
    const RowMap rm{ws.grp.order, x_rows, 1, x_row_count, &ws.hdr->status};
    const int max_active = (int)(rows < num_experts ? rows : num_experts);
    if (bits == 4 && rows <= gemv_threshold() && k_in <= 2048)
      launch_gemv_plain(dtype == TFM_DTYPE_F16, static_cast<const uint16_t*>(x), rm, ws.grp, max_active, rows, *w, n_out, k_in,
                        static_cast<uint16_t*>(out), s);
    else
      launch_ggemm_plain(static_cast<const uint16_t*>(x), rm, ws.grp, rows, num_experts, *w, n_out,
                         k_in, bits, dtype == TFM_DTYPE_F16, static_cast<uint16_t*>(out), s);
  });
}

int tfm_affine_qmm(const void* x, int64_t rows, const tfm_affine* w, int32_t n_out,
                   int32_t k_in, int32_t group_size, int32_t bits, int32_t dtype, void* out,
                   void* stream) {
  return guarded([&] {
    need(rows >= 0 && rows <= INT32_MAX, "rows out of range");
    need(n_out > 0 && k_in > 0, "n_out and k_in must be positive");
    need(bits == 4 || bits == 8, "bits must be 4 or 8");
    need(group_size == 32 || group_size == 64 || group_size == 128, "group_size must be 32, 64 or 128");
    need(k_in % group_size == 0, "k_in must be a multiple of group_size");
    if (group_size != 64) fail(TFM_E_UNSUPPORTED, "only group_size 64 is built");
    need(dtype == TFM_DTYPE_BF16 || dtype == TFM_DTYPE_F16, "unknown dtype");
    if (n_out % 64 != 0) fail(TFM_E_UNSUPPORTED, "n_out must be a multiple of 64");
    if (rows == 0) return;
    need_ptr(x, "x");
    need_ptr(w, "w");
    need_ptr(out, "out");
    need_align16(x, "x");
    check_affine(*w, "w");
    hipStream_t s = static_cast<hipStream_t>(stream);
    // One expert owning every row in caller order: no grouping pass, and no
    // row can be out of range (the status word is never written).
    Grouping grp{};
    grp.E = 1;
    grp.ident = (int)rows;
    const RowMap rm{nullptr, nullptr, 1, rows, nullptr};
    if (bits == 4 && rows <= gemv_threshold() && k_in <= 2048)
      launch_gemv_plain(dtype == TFM_DTYPE_F16, static_cast<const uint16_t*>(x), rm, grp, 1, rows, *w, n_out, k_in,
                        static_cast<uint16_t*>(out), s);
    else
      launch_ggemm_plain(static_cast<const uint16_t*>(x), rm, grp, rows, 1, *w, n_out, k_in, bits,
                         dtype == TFM_DTYPE_F16, static_cast<uint16_t*>(out), s);
  });
}

int tfm_moe_experts(const tfm_plan* plan, const void* x, int64_t tokens, const void* residual,
                    const int32_t* idx, const float* gates, const tfm_moe_weights* weights, void* y,
                    uint32_t flags, void* workspace, size_t workspace_bytes, void* stream) {
  return guarded([&] {
    need_ptr(plan, "plan");
    need(tokens >= 0 && tokens <= INT32_MAX / 64, "tokens out of range");
    if (tokens == 0) return;
    need_ptr(x, "x");
    need_ptr(idx, "idx");
    need_ptr(gates, "gates");
    need_ptr(y, "y");
    need_align16(x, "x");
    need_align16(y, "y");
    if (residual) need_align16(residual, "residual");
    check_weights(weights, false, plan->g);
    BlockWs ws = carve_block(plan->g, tokens, workspace);
    need_ws(workspace, workspace_bytes, ws.bytes);
    run_experts(plan, static_cast<const uint16_t*>(x), tokens, static_cast<const uint16_t*>(residual),
                idx, gates, weights, static_cast<uint16_t*>(y), flags, ws,
                static_cast<hipStream_t>(stream));
  });
}

// The block on x (already in the layer's dtype and shape): routing, grouping,
// experts, combine with `residual` (may be null). Inputs are validated by
// the entry points.
static void moe_forward_body(const tfm_plan* plan, const void* x, int64_t tokens, const void* residual,
                             const tfm_moe_weights* weights, void* y, int32_t* idx_out, float* gates_out,
                             uint32_t flags, BlockWs& ws, hipStream_t s) {
  const tfm_geometry& g = plan->g;
  const int64_t R = tokens * g.experts_per_token;
  const int T = (int)tokens, E = g.num_experts, K = g.experts_per_token;
  const int H = g.hidden_size, I = g.intermediate_size;
  const bool f16 = g.dtype == TFM_DTYPE_F16;
  const DecodeChoice dc = decode_choice(g, R, plan->gemv_max_routes);
  const bool gemv_decode = dc.gemv;
  if (dc.stream) {
    Grouping gd = ws.grp;
    gd.slots = ws.slots;
    gd.gates_sorted = ws.gates_sorted;
    {
      // An affine router is dequantised inside the logits kernel.
      StageScope st(TFM_STAGE_ROUTER, s);
      if (g.router != TFM_ROUTER_AFFINE ||
          !launch_decode_logits_affine(f16, weights->router_bits, static_cast<const uint16_t*>(x),
                                       weights->router_affine, weights->logit_bias, T, H, E, ws.logits, s)) {
        const uint16_t* rw = static_cast<const uint16_t*>(weights->router);
        if (g.router == TFM_ROUTER_AFFINE) {
          launch_dequant_router(f16, weights->router_bits, weights->router_affine, E, H, ws.router_w, s);
          rw = ws.router_w;
        }
        launch_decode_logits(f16, static_cast<const uint16_t*>(x), rw, weights->logit_bias, T, H, E, ws.logits, s);
      }
    }
    {
      // Top-k and grouping run in this kernel's prologue.
      StageScope st(TFM_STAGE_GATEUP, s);
      launch_ds_gateup(f16, g.bits, g.route, static_cast<const uint16_t*>(x), ws.logits, ws.idx, ws.gates, T, K, E, H,
                       I, weights->gate, weights->up, gd, &ws.hdr->status, ws.h, s,
                       ds_prefetch() ? &weights->down : nullptr);
    }
    const int max_active = (int)(R < E ? R : E);
    if (decode_small(T, K)) {
      StageScope st(TFM_STAGE_DOWN, s);
      launch_ds_down_combine(f16, g.bits, ws.h, ds_h_route_order(g.route, T, K), ws.idx, ws.gates, ws.grp.inverse,
                             T, K, E, H, I, weights->down,
                             static_cast<const uint16_t*>(residual), g.residual_multiplier,
                             static_cast<uint16_t*>(y), s);
    } else {
      {
        StageScope st(TFM_STAGE_DOWN, s);
        launch_ds_down(f16, g.bits, ws.h, H, I, max_active, weights->down, gd, ws.P, s);
      }
      StageScope st(TFM_STAGE_COMBINE, s);
      launch_combine_sorted(f16, ws.P, ws.grp.inverse, ws.grp.offsets + E, T, K, H,
                            static_cast<const uint16_t*>(residual), g.residual_multiplier,
                            static_cast<uint16_t*>(y), s);
    }
    if (idx_out) launch_copy_i32(ws.idx, idx_out, R, s);
    if (gates_out) launch_copy_i32(reinterpret_cast<const int32_t*>(ws.gates),
                                   reinterpret_cast<int32_t*>(gates_out), R, s);
    return;
  }
  if (gemv_decode) {
    {
      StageScope st(TFM_STAGE_ROUTER, s);
      if (g.router == TFM_ROUTER_AFFINE &&
          launch_decode_logits_affine(f16, weights->router_bits, static_cast<const uint16_t*>(x),
                                      weights->router_affine, weights->logit_bias, T, H, E, ws.logits, s)) {
        // An affine router is dequantised inside the logits kernel.
      } else {
        const uint16_t* rw = static_cast<const uint16_t*>(weights->router);
        if (g.router == TFM_ROUTER_AFFINE) {
          launch_dequant_router(f16, weights->router_bits, weights->router_affine, E, H, ws.router_w, s);
          rw = ws.router_w;
        }
        launch_decode_logits(f16, static_cast<const uint16_t*>(x), rw, weights->logit_bias, T, H, E, ws.logits, s);
      }
    }
    Grouping gd = ws.grp;
    gd.slots = ws.slots;
    gd.gates_sorted = ws.gates_sorted;
    if (decode_slot_grouping(T, K, E, H, I)) {
      // One workgroup ranks and groups the routes and publishes the slot
      // table; every gate/up workgroup then reads its slot.
      {
        StageScope st(TFM_STAGE_TOPK, s);
        launch_ds_route_group(f16, g.route, ws.logits, T, E, K, ws.idx, ws.gates, gd, &ws.hdr->status, s);
      }
      StageScope st(TFM_STAGE_GATEUP, s);
      const RowMap rmx{gd.order, nullptr, K, T, &ws.hdr->status};
      launch_gemv_gateup(f16, static_cast<const uint16_t*>(x), rmx, gd, (int)(R < E ? R : E), R,
                         weights->gate, weights->up, I, H, ws.h, s);
    } else {
      // Top-k over many workgroups; every gate/up workgroup groups the routes
      // itself, and its first publishes the grouping for the down GEMV.
      {
        StageScope st(TFM_STAGE_TOPK, s);
        launch_topk(g.route, f16, ws.logits, T, E, K, ws.idx, nullptr, ws.gates, s);
      }
      StageScope st(TFM_STAGE_GATEUP, s);
      launch_decode_gateup(f16, static_cast<const uint16_t*>(x), ws.idx, ws.gates, T, E, K, H, I,
                           weights->gate, weights->up, gd, ws.h, &ws.hdr->status, s);
    }
    const int max_active = (int)(R < E ? R : E);
    {
      StageScope st(TFM_STAGE_DOWN, s);
      launch_gemv_scaled(f16, ws.h, gd, max_active, R, weights->down, H, I, ws.gates, ws.P, s);
    }
    {
      StageScope st(TFM_STAGE_COMBINE, s);
      launch_combine_sorted(f16, ws.P, ws.grp.inverse, ws.grp.offsets + E, T, K, H,
                            static_cast<const uint16_t*>(residual), g.residual_multiplier,
                            static_cast<uint16_t*>(y), s);
    }
    if (idx_out) launch_copy_i32(ws.idx, idx_out, R, s);
    if (gates_out) launch_copy_i32(reinterpret_cast<const int32_t*>(ws.gates),
                                   reinterpret_cast<int32_t*>(gates_out), R, s);
    return;
  }

  bool fused_route = false;
  {
    // Router linear, top-k and chunk histograms in one kernel where the
    // hidden size has a variant; otherwise logits then top-k. An affine
    // router is first dequantised to a dense matrix in the workspace.
    StageScope st(TFM_STAGE_ROUTER, s);
    const uint16_t* rw = static_cast<const uint16_t*>(weights->router);
    if (g.router == TFM_ROUTER_AFFINE) {
      launch_dequant_router(f16, weights->router_bits, weights->router_affine, E, H, ws.router_w, s);
      rw = ws.router_w;
    }
    if (T > router_split_max_tokens())
      fused_route = launch_router_topk(g.route, f16, static_cast<const uint16_t*>(x), rw, weights->logit_bias,
                                       T, H, E, K, ws.idx, ws.gates, ws.hist, nullptr, s);
    if (!fused_route)
      launch_router_logits(f16, static_cast<const uint16_t*>(x), rw, weights->logit_bias, (int)tokens, H, E,
                           ws.logits, s);
  }
  // At most 256 routes: top-k and grouping in one workgroup (the streaming
  // decode kernels' routing and grouping), one kernel instead of three.
  const bool small_group = !fused_route && R <= 256;
  if (small_group) {
    StageScope st(TFM_STAGE_TOPK, s);
    Grouping gd = ws.grp;
    gd.slots = ws.slots;
    gd.gates_sorted = ws.gates_sorted;
    launch_ds_route_group(f16, g.route, ws.logits, T, E, K, ws.idx, ws.gates, gd, &ws.hdr->status, s);
  } else if (!fused_route) {
    StageScope st(TFM_STAGE_TOPK, s);
    launch_topk_hist(g.route, f16, ws.logits, T, E, K, ws.idx, ws.gates, ws.hist, s);
  }
  if (!small_group) {
    StageScope st(TFM_STAGE_GROUP, s);
    launch_group_scatter(ws.idx, R, E, kTopkTokensPerBlock * K, ws.hist, ws.grp, &ws.hdr->status, s);
  }
  if (idx_out) launch_copy_i32(ws.idx, idx_out, R, s);
  if (gates_out) launch_copy_i32(reinterpret_cast<const int32_t*>(ws.gates),
                                 reinterpret_cast<int32_t*>(gates_out), R, s);
  run_experts(plan, static_cast<const uint16_t*>(x), tokens, static_cast<const uint16_t*>(residual),
              ws.idx, ws.gates, weights, static_cast<uint16_t*>(y), flags, ws, s, true);
}

int tfm_moe_forward(const tfm_plan* plan, const void* x, int64_t tokens, const void* residual,
                    const tfm_moe_weights* weights, void* y, int32_t* idx_out, float* gates_out,
                    uint32_t flags, void* workspace, size_t workspace_bytes, void* stream) {
  return guarded([&] {
    need_ptr(plan, "plan");
    need(tokens >= 0 && tokens <= INT32_MAX / 64, "tokens out of range");
    if (tokens == 0) return;
    need_ptr(x, "x");
    need_ptr(y, "y");
    need_align16(x, "x");
    need_align16(y, "y");
    if (residual) need_align16(residual, "residual");
    check_weights(weights, true, plan->g);
    BlockWs ws = carve_block(plan->g, tokens, workspace);
    need_ws(workspace, workspace_bytes, ws.bytes);
    moe_forward_body(plan, x, tokens, residual, weights, y, idx_out, gates_out, flags, ws,
                     static_cast<hipStream_t>(stream));
  });
}

int tfm_moe_forward_static(const tfm_plan* plan, const void* x, int64_t tokens, const void* residual,
                           const tfm_moe_weights* weights, void* y, int32_t* idx_out, float* gates_out,
                           uint32_t flags, void* stream) {
  return guarded([&] {
    need_ptr(plan, "plan");
    need(tokens >= 0 && tokens <= INT32_MAX / 64, "tokens out of range");
    if (tokens == 0) return;
    need_ptr(x, "x");
    need_ptr(y, "y");
    need_align16(x, "x");
    need_align16(y, "y");
    if (residual) need_align16(residual, "residual");
    check_weights(weights, true, plan->g);
    const size_t want = carve_block(plan->g, tokens, nullptr).bytes;
    if (want > kStaticScratchBytes)
      fail(TFM_E_WORKSPACE, "tfm_moe_forward_static: " + std::to_string(tokens) + " tokens need " +
                                std::to_string(want) + " bytes of scratch, more than the static array's " +
                                std::to_string(kStaticScratchBytes) + " (use tfm_moe_forward with a workspace)");
    if (!plan->scratch)
      fail(TFM_E_HIP, "tfm_moe_forward_static: no static scratch on the plan's device (" + plan->scratch_error + ")");
    BlockWs ws = carve_block(plan->g, tokens, plan->scratch);
    moe_forward_body(plan, x, tokens, residual, weights, y, idx_out, gates_out, flags, ws,
                     static_cast<hipStream_t>(stream));
  });
}

int tfm_moe_forward_rmsnorm(const tfm_plan* plan, const void* h, int64_t tokens, const void* norm_weight,
                            float eps, const tfm_moe_weights* weights, void* y, int32_t* idx_out,
                            float* gates_out, uint32_t flags, void* workspace, size_t workspace_bytes,
                            void* stream) {
  return guarded([&] {
    need_ptr(plan, "plan");
    need(tokens >= 0 && tokens <= INT32_MAX / 64, "tokens out of range");
    need(eps >= 0.0f && eps == eps, "eps must be a non-negative number");
    if (tokens == 0) return;
    need_ptr(h, "h");
    need_ptr(norm_weight, "norm_weight");
    need_ptr(y, "y");
    need_align16(h, "h");
    need_align16(norm_weight, "norm_weight");
    need_align16(y, "y");
    need(y != h, "y must not alias h (h is the residual)");
    check_weights(weights, true, plan->g);
    BlockWs ws = carve_block(plan->g, tokens, workspace);
    need_ws(workspace, workspace_bytes, ws.bytes);
    hipStream_t s = static_cast<hipStream_t>(stream);
    {
      StageScope st(TFM_STAGE_NORM, s);
      launch_rmsnorm(plan->g.dtype == TFM_DTYPE_F16, static_cast<const uint16_t*>(h), static_cast<const uint16_t*>(norm_weight), eps,
                     (int)tokens, plan->g.hidden_size, ws.xn, s);
    }
    moe_forward_body(plan, ws.xn, tokens, h, weights, y, idx_out, gates_out, flags, ws, s);
  });
}

size_t tfm_expert_routes_workspace_bytes(const tfm_plan* plan, int64_t n_routes) {
  if (!plan || n_routes < 0) return 0;
  const tfm_geometry& g = plan->g;
  Carver c(nullptr);
  c.take<WsHeader>(1);
  c.take<int32_t>((size_t)n_routes);           // order
  c.take<int32_t>((size_t)g.num_experts + 1);  // offsets
  c.take<int32_t>((size_t)g.num_experts + 1);  // active
  c.take<uint16_t>((size_t)(n_routes * g.intermediate_size));
  c.take<float>((size_t)(n_routes * g.hidden_size));
  c.take<int32_t>((size_t)group_hist_rows(group_blocks(n_routes, kGroupChunk)) * (g.num_experts + 1));
  return align_up(c.offset, 256);
}

int tfm_expert_routes(const tfm_plan* plan, const void* x, int64_t tokens,
                      const int32_t* token_indices, const int32_t* expert_ids, int64_t n_routes,
                      int32_t experts_sorted, const tfm_moe_weights* weights, void* out_sorted,
                      int32_t* inverse, void* workspace, size_t workspace_bytes, void* stream) {
  (void)experts_sorted;
  return guarded([&] {
    need_ptr(plan, "plan");
    need(tokens >= 0 && tokens <= INT32_MAX, "tokens out of range");
    need(n_routes >= 0 && n_routes <= INT32_MAX, "n_routes out of range");
    const tfm_geometry& g = plan->g;
    const size_t want = tfm_expert_routes_workspace_bytes(plan, n_routes);
    need_ws(workspace, workspace_bytes, want);
    if (n_routes == 0) return;
    need(tokens > 0, "routes given but x has no tokens");
    need_ptr(x, "x");
    need_ptr(token_indices, "token_indices");
    need_ptr(expert_ids, "expert_ids");
    need_ptr(out_sorted, "out_sorted");
    need_ptr(inverse, "inverse");
    need_align16(x, "x");
    check_weights(weights, false, plan->g);
    Carver c(workspace);
    WsHeader* hdr = c.take<WsHeader>(1);
    Grouping grp{};
    grp.order = c.take<int32_t>((size_t)n_routes);
    grp.offsets = c.take<int32_t>((size_t)g.num_experts + 1);
    grp.active = c.take<int32_t>((size_t)g.num_experts + 1);
    grp.inverse = inverse;
    grp.E = g.num_experts;
    uint16_t* h = c.take<uint16_t>((size_t)(n_routes * g.intermediate_size));
    float* P = c.take<float>((size_t)(n_routes * g.hidden_size));
    int32_t* hist = c.take<int32_t>((size_t)group_hist_rows(group_blocks(n_routes, kGroupChunk)) * (g.num_experts + 1));
    hipStream_t s = static_cast<hipStream_t>(stream);
    const int H = g.hidden_size, I = g.intermediate_size, E = g.num_experts;
    launch_group(expert_ids, n_routes, E, grp, hist, &hdr->status, s);
    const RowMap rm{grp.order, token_indices, 1, tokens, &hdr->status};
    const int max_active = (int)(n_routes < E ? n_routes : E);
    const uint16_t* xp = static_cast<const uint16_t*>(x);
    const bool f16 = g.dtype == TFM_DTYPE_F16;
    if (n_routes <= plan->gemv_max_routes && H <= 2048 && I <= 2048 && g.bits == 4) {
      launch_gemv_gateup(f16, xp, rm, grp, max_active, n_routes, weights->gate, weights->up, I, H, h, s);
      launch_gemv_scaled(f16, h, grp, max_active, n_routes, weights->down, H, I, nullptr, P, s);
      launch_rows_to_st(f16, P, n_routes, H, static_cast<uint16_t*>(out_sorted), s);
    } else {
      launch_ggemm_gateup(xp, rm, grp, n_routes, E, weights->gate, weights->up, I, H, g.bits, f16, h, s);
      launch_ggemm_down(h, grp, n_routes, E, weights->down, H, I, g.bits, f16,
                        static_cast<uint16_t*>(out_sorted), s);
    }
  });
}

int tfm_profiler_create(int32_t capacity, tfm_profiler** out) {
  return guarded([&] {
    need_ptr(out, "out");
    *out = nullptr;
    need(capacity > 0 && capacity <= (1 << 20), "capacity must be in [1, 2^20]");
    tfm_profiler* p = new tfm_profiler{};
    p->capacity = capacity;
    p->start.assign((size_t)capacity, nullptr);
    p->end.assign((size_t)capacity, nullptr);
    p->stage.assign((size_t)capacity, -1);
    p->kernel.assign((size_t)capacity, KernelTimer{});
    for (int i = 0; i < capacity; ++i) {
      hipError_t err = hipEventCreate(&p->start[i]);
      if (err == hipSuccess) err = hipEventCreate(&p->end[i]);
      if (err == hipSuccess) err = hipEventCreate(&p->kernel[i].start);
      if (err == hipSuccess) err = hipEventCreate(&p->kernel[i].end);
      if (err != hipSuccess) {
        tfm_profiler_destroy(p);
        check_hip(err, "hipEventCreate");
      }
    }
    *out = p;
  });
}

void tfm_profiler_destroy(tfm_profiler* p) {
  if (!p) return;
  if (g_profiler == p) g_profiler = nullptr;
  for (hipEvent_t e : p->start)
    if (e) (void)hipEventDestroy(e);
  for (hipEvent_t e : p->end)
    if (e) (void)hipEventDestroy(e);
  for (const KernelTimer& k : p->kernel) {
    if (k.start) (void)hipEventDestroy(k.start);
    if (k.end) (void)hipEventDestroy(k.end);
  }
  delete p;
}

int tfm_profiler_attach(tfm_profiler* p) {
  g_profiler = p;
  g_kernel_timer = nullptr;
  return TFM_OK;
}

int tfm_profiler_reset(tfm_profiler* p) {
  return guarded([&] {
    need_ptr(p, "profiler");
    p->used = 0;
    p->dropped = 0;
  });
}

int tfm_profiler_stage(tfm_profiler* p, int32_t stage, double* total_ms, int32_t* launches,
                       int32_t* dropped) {
  return guarded([&] {
    need_ptr(p, "profiler");
    need(stage >= 0 && stage < TFM_STAGE_COUNT, "unknown stage");
    double sum = 0.0;
    int n = 0;
    for (int i = 0; i < p->used; ++i) {
      if (p->stage[i] != stage) continue;
      check_hip(hipEventSynchronize(p->end[i]), "hipEventSynchronize");
      float ms = 0.0f;
      check_hip(hipEventElapsedTime(&ms, p->start[i], p->end[i]), "hipEventElapsedTime");
      sum += ms;
      ++n;
    }
    if (total_ms) *total_ms = sum;
    if (launches) *launches = n;
    if (dropped) *dropped = p->dropped;
  });
}

int tfm_profiler_stage_kernel(tfm_profiler* p, int32_t stage, double* kernel_ms, int32_t* kernels) {
  return guarded([&] {
    need_ptr(p, "profiler");
    need(stage >= 0 && stage < TFM_STAGE_COUNT, "unknown stage");
    double sum = 0.0;
    int n = 0;
    for (int i = 0; i < p->used; ++i) {
      if (p->stage[i] != stage || !p->kernel[i].used) continue;
      check_hip(hipEventSynchronize(p->kernel[i].end), "hipEventSynchronize");
      float ms = 0.0f;
      check_hip(hipEventElapsedTime(&ms, p->kernel[i].start, p->kernel[i].end), "hipEventElapsedTime");
      sum += ms;
      ++n;
    }
    if (kernel_ms) *kernel_ms = sum;
    if (kernels) *kernels = n;
  });
}

const char* tfm_stage_name(int32_t stage) {
  static const char* names[TFM_STAGE_COUNT] = {"router", "topk", "group", "gateup", "down", "combine",
                                               "norm"};
  return stage >= 0 && stage < TFM_STAGE_COUNT ? names[stage] : "";
}

int tfm_status_word(void* workspace, void* stream, uint32_t* status_out) {
  return guarded([&] {
    need_ptr(workspace, "workspace");
    need_ptr(status_out, "status_out");
    hipStream_t s = static_cast<hipStream_t>(stream);
    WsHeader* hdr = static_cast<WsHeader*>(workspace);
    uint32_t v = 0;
    check_hip(hipMemcpyAsync(&v, &hdr->status, sizeof(v), hipMemcpyDeviceToHost, s), "status read");
    check_hip(hipStreamSynchronize(s), "status sync");
    const uint32_t zero = 0;
    check_hip(hipMemcpyAsync(&hdr->status, &zero, sizeof(zero), hipMemcpyHostToDevice, s), "status clear");
    check_hip(hipStreamSynchronize(s), "status sync");
    *status_out = v;
  });
}

}  // extern "C"
