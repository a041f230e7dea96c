// Decode path, streaming form (few routes: T*K <= 256, small T).
//
// The block NativeGraniteMoEPrefill::moe runs per layer
// (MLXNativeGraniteMoEPrefill.h:627-702) at decode shapes, as five kernels:
//   1. decode_logits_kernel (decode.hip): router logits, one workgroup per expert,
//   2. ds_topk_group_kernel: one workgroup ranks every token (OLMoE or Granite
//      rules, route_wave.h) and groups the T*K routes by expert (stable), then
//      publishes the grouping, a slot table {expert, first route, end route}
//      and the active-slot count,
//   3. ds_gateup_kernel: dequant GEMV of gate and up with the SwiGLU epilogue,
//   4. ds_down_kernel: dequant GEMV of down, scaled by each route's gate (fp32),
//   5. combine_sorted_kernel (combine.hip): ordered K reduction + residual.
//
// Work split of the two GEMV kernels. An item is a few rows of one routed
// expert (4 rows per wave-wide load: 16 lanes per row, each lane owning
// 32-element chunks 16c + l of the row, one 16-byte load per chunk). Items
// are ordered (active slot, row block) and every wave takes a contiguous range
// of them, cut by cost (a fixed share for the nibble unpack plus one share per
// route of the expert), so hot experts do not leave a tail. A wave loads its
// range's slot data once, issues the loads of its next item before it reduces
// and stores the current one, and never waits on another wave after the
// start: gate/up stages the x rows of all T tokens once per workgroup; down
// stages the h rows of the current expert's routes per wave.
//
// Arithmetic per chunk (inside one 64-wide group) as in the other GEMVs:
//   sum_k x_k (s q_k + b) = s * sum_k x_k (128 + q_k) + (b - 128 s) * sum_k x_k,
// with (128 + q) built exactly in bf16 by byte permutes and the products run
// as v_dot2_f32_bf16 with fp32 accumulation (no MFMA).
#include <algorithm>
#include <cstdlib>

#include "gemv_body.h"
#include "route_wave.h"

// Compiled twice: as is for bf16 storage (namespace tfm::ds_bf16) and from
// dstream_f16.hip for IEEE-half storage (tfm::ds_f16). Only the arithmetic on
// 16-bit values differs: conversions, the dot2 instruction, the exponent
// byte of the unpacked codes and the matching code base.
#ifndef TFM_DS_F16
#define TFM_DS_F16 0
#endif
#ifndef TFM_DS_BITS
#define TFM_DS_BITS 4
#endif
#if TFM_DS_F16 && TFM_DS_BITS == 8
#define TFM_DS_NS ds_f16_i8
#elif TFM_DS_F16
#define TFM_DS_NS ds_f16
#elif TFM_DS_BITS == 8
#define TFM_DS_NS ds_bf16_i8
#else
#define TFM_DS_NS ds_bf16
#endif

namespace tfm {
namespace TFM_DS_NS {

constexpr bool kF16 = TFM_DS_F16 != 0;
// Code width. A 32-element chunk is 16 bytes of nibbles (4-bit) or 32 bytes
// of byte codes (8-bit). An 8-bit code c = lo + 16 hi is dotted as its two
// nibbles with the same (base + nibble) trick: sum x (base+lo) + 16 sum x
// (base+hi) = sum x c + 17 base sum x.
constexpr int kBits = TFM_DS_BITS;
static_assert(kBits == 4 || kBits == 8, "4-bit or 8-bit codes");
constexpr int kQW = kBits / 4;  // 16-byte loads per 32-element chunk
__host__ __device__ constexpr float code_corr() { return (kBits == 4 ? 1.0f : 17.0f) * code_base(kF16); }

constexpr int kDsCostUnpack = 2;  // item cost = kDsCostUnpack + routes of its expert
constexpr int kDsDownXB = 4;      // h rows staged per wave in the down kernel

__device__ __forceinline__ int readlane_i(int v, int l) { return __builtin_amdgcn_readlane(v, l); }
// Marks a wave-uniform value as such, so that buffer resources built from it
// stay in scalar registers.
__device__ __forceinline__ int uni(int v) { return __builtin_amdgcn_readfirstlane(v); }

// Inclusive prefix sum over the 64 lanes of a wave.
__device__ __forceinline__ int wave_incl_scan(int v) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const int o = __shfl_up(v, d, 64);
    if (lane >= d) v += o;
  }
  return v;
}

// Slot data of the active experts (one slot per lane; the slot table also
// carries the active count in .w) and the contiguous range [i0, i1) of flat
// item indices i = slot * ipe + row block of wave `gw` of `nw` waves. The
// range is cut by cost, item cost = kDsCostUnpack + routes of its slot: the
// wave takes the items whose start cost lies in [gw, gw+1) * total / nw.
struct WaveRange {
  int4 sl;     // this lane's slot {expert, first route, end route, active count}
  int ipe;     // items (row blocks) per expert
  int i0, i1;  // flat item range
};

__device__ __forceinline__ int4 load_slot(const int4* __restrict__ slots, int E) {
  const int lane = threadIdx.x & 63;
  return lane < E ? slots[lane] : make_int4(-1, 0, 0, 0);
}

// sl: load_slot's result (lane 0's slot always exists, E >= 1).
__device__ __forceinline__ void wave_range(int4 sl, int ipe, int gw, int nw, WaveRange& w) {
  const int lane = threadIdx.x & 63;
  w.ipe = ipe;
  w.sl = sl;
  const int U = uni(w.sl.w);
  const bool on = lane < U;
  const int rl = on ? w.sl.z - w.sl.y : 0;
  const int cost = on ? ipe * (kDsCostUnpack + rl) : 0;
  const int incl = wave_incl_scan(cost);
  const int total = readlane_i(incl, 63);
  const int c0 = (int)((int64_t)gw * total / nw);
  const int c1 = (int)((int64_t)(gw + 1) * total / nw);
  // First item whose start cost is >= c: its slot is the count of slots whose
  // inclusive cost is <= c; within the slot, start cost = excl + r * weight.
  auto first = [&](int c) -> int {
    const int a = __popcll(__ballot(on && incl <= c));
    if (a >= U) return U * ipe;
    const int excl = readlane_i(incl - cost, a);
    const int wgt = kDsCostUnpack + readlane_i(rl, a);
    const int rr = (c - excl + wgt - 1) / wgt;
    return rr >= ipe ? (a + 1) * ipe : a * ipe + rr;
  };
  w.i0 = uni(first(c0));
  w.i1 = uni(first(c1));
}

// ---------------------------------------------------------------------------
// 2. Routing and grouping (in the gate/up kernel's prologue).
constexpr int kDsGiven = kDsGivenRoutes;  // routes given (idx, fp32 gates) instead of ranked

// LDS of the in-workgroup routing and grouping.
struct DsGroupLds {
  int e[256];       // route -> bucket (expert, E for a bad id)
  float g[256];     // route -> fp32 gate
  int wcnt[4][65];  // per grouping wave: routes per bucket
  int wpre[4][65];  // per grouping wave: first position per bucket
  int off[66];      // bucket offsets
  int act[65];      // active experts ascending; act[E] = count
  int order[256];   // sorted position -> flat route
};

// Routing and stable grouping of the T*K routes of every token, inside one
// workgroup of at least 4 waves (R = T*K <= 256). MODE OLMOE/GRANITE ranks
// the logits [T, E] (route_wave.h; waves take tokens round-robin); kDsGiven
// takes the routes (ids and fp32 gates) from idx/gates instead: ids outside
// [0, E) sort after every valid id (bucket E), are left out of the active
// list and set TFM_STATUS_BAD_EXPERT_ID. The position of route f is the
// number of routes to lower buckets plus the routes to its bucket with a
// lower flat index. Results land in L (the caller synchronises before reading
// them); with `publish`, also in the workspace: flat idx/gates (ranked
// modes), order, inverse, offsets, active list, sorted gates, the slot table
// {expert, first route, end route, active count} and the status word.
template <int MODE>
__device__ __forceinline__ void ds_rank_group(DsGroupLds& L, const uint16_t* __restrict__ logits, int T,
                                              int E, int K, int32_t* __restrict__ idx,
                                              float* __restrict__ gates, bool publish, const Grouping& g,
                                              uint32_t* __restrict__ status) {
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int nwaves = blockDim.x >> 6;
  const int R = T * K;
  if (MODE == kDsGiven) {
    if (tid < R) {
      const int id = idx[tid];
      L.e[tid] = (id < 0 || id >= E) ? E : id;
      L.g[tid] = gates[tid];
    }
  } else {
    for (int t = wave; t < T; t += nwaves) {
      const uint16_t* row = logits + (int64_t)t * E;
      float gv;
      int id;
      if (MODE == TFM_ROUTE_OLMOE) {
        uint16_t gb;
        id = olmoe_route_wave<kF16>(row, E, K, &gv, &gb);
      } else {
        id = granite_route_wave<kF16>(row, E, K, &gv);
      }
      if (lane < K) {
        L.e[t * K + lane] = id;
        L.g[t * K + lane] = gv;
        if (publish) {
          idx[(int64_t)t * K + lane] = id;
          gates[(int64_t)t * K + lane] = gv;
        }
      }
    }
  }
  for (int i = tid; i < 4 * 65; i += blockDim.x) (&L.wcnt[0][0])[i] = 0;
  __syncthreads();
  const bool live = tid < R;
  const int e = live ? L.e[tid] : 0;
  int rank_w = 0;
  if (wave < 4) {
    uint64_t match = __ballot(live);
#pragma unroll
    for (int bit = 0; bit < 7; ++bit) {
      const bool b = (e >> bit) & 1;
      const uint64_t ones = __ballot(live && b);
      match &= b ? ones : ~ones;
    }
    const uint64_t lt = lane == 0 ? 0ull : (~0ull >> (64 - lane));
    rank_w = __popcll(match & lt);
    if (live && rank_w == 0) L.wcnt[wave][e] = __popcll(match);
  }
  __syncthreads();
  if (wave == 0) {
    // Lanes 0..63 hold experts 0..63; the bad bucket E (<= 64) comes last.
    const int c0 = L.wcnt[0][lane], c1 = L.wcnt[1][lane], c2 = L.wcnt[2][lane], c3 = L.wcnt[3][lane];
    const int cnt = lane < E ? c0 + c1 + c2 + c3 : 0;
    const int incl = wave_incl_scan(cnt);
    const int excl = incl - cnt;
    if (lane < E) {
      L.off[lane] = excl;
      L.wpre[0][lane] = excl;
      L.wpre[1][lane] = excl + c0;
      L.wpre[2][lane] = excl + c0 + c1;
      L.wpre[3][lane] = excl + c0 + c1 + c2;
    }
    if (lane == 63) {
      L.off[E] = incl;
      int b = incl;
      L.wpre[0][E] = b; b += L.wcnt[0][E];
      L.wpre[1][E] = b; b += L.wcnt[1][E];
      L.wpre[2][E] = b; b += L.wcnt[2][E];
      L.wpre[3][E] = b;
      L.off[E + 1] = b + L.wcnt[3][E];  // == R
    }
    const uint64_t act = __ballot(lane < E && cnt > 0);
    const uint64_t lt = lane == 0 ? 0ull : (~0ull >> (64 - lane));
    if (lane < E && cnt > 0) L.act[__popcll(act & lt)] = lane;
    if (lane == 0) L.act[E] = __popcll(act);
  }
  __syncthreads();
  if (live) {
    const int pos = L.wpre[wave][e] + rank_w;
    L.order[pos] = tid;
    if (publish) {
      g.order[pos] = tid;
      g.inverse[tid] = pos;
      g.gates_sorted[pos] = L.g[tid];
    }
  }
  if (publish) {
    const int U = L.act[E];
    if (tid <= E) {
      g.offsets[tid] = L.off[tid];
      if (tid == E || tid < U) g.active[tid] = L.act[tid];
    }
    if (tid < E) {
      const int ex = tid < U ? L.act[tid] : -1;
      g.slots[tid] = ex < 0 ? make_int4(-1, 0, 0, U) : make_int4(ex, L.off[ex], L.off[ex + 1], U);
    }
    // Sticky: bits accumulate until tfm_status_word reads and clears them.
    if (tid == 0 && L.off[E] < R) atomicOr(status, (uint32_t)TFM_STATUS_BAD_EXPERT_ID);
  }
}

// Routing and grouping alone (the prefill path's top-k and grouping for at
// most 256 routes): one workgroup of 16 waves, each ranking every 16th token,
// then ds_rank_group's grouping, published. One kernel instead of the top-k
// and scatter kernels of larger batches.
template <int MODE>
__global__ __launch_bounds__(1024) void ds_route_group_kernel(const uint16_t* __restrict__ logits, int T, int E,
                                                              int K, int32_t* __restrict__ idx,
                                                              float* __restrict__ gates, Grouping g,
                                                              uint32_t* __restrict__ status) {
  __shared__ DsGroupLds L;
  ds_rank_group<MODE>(L, logits, T, E, K, idx, gates, true, g, status);
}

// ---------------------------------------------------------------------------
// Raw loads of one row for lane column ll: its C chunks of packed codes
// (chunk c: elements 32 (16c + ll) .. + 31, in group 8c + ll / 2) and one
// dword each of the row's scales and biases. The 16 lanes of a row read its
// group scales as 16 dwords in one instruction: lane ll reads dword
// 4 (ll % 4) + ll / 4, so lane 4Q + c of quad Q holds dword 4c + Q, the
// groups 8c + 2Q and 8c + 2Q + 1 that the lanes of quad Q use for chunk c
// (ds_row_sb hands them out with one quad broadcast). Two loads per row
// instead of one per chunk: a third fewer memory requests per item. Rows
// narrower than 2048 leave some dwords unused (they read the next row or
// zeros past the buffer).
template <int C>
struct DsRow {
  uint4 q[C][kQW];
  uint32_t s, b;
};

struct DsMat {
  __amdgpu_buffer_rsrc_t q, s, b;
};

// Buffer resources over expert e's rows of one matrix; rows >= N read zero.
__device__ __forceinline__ DsMat ds_mat(const tfm_affine& m, int e, int N, int kin) {
  const uint32_t qrow = (uint32_t)kin * kBits / 8, srow = (uint32_t)kin / 32;
  DsMat d;
  d.q = make_rsrc(reinterpret_cast<const char*>(m.q) + (size_t)e * N * qrow, (uint32_t)N * qrow);
  d.s = make_rsrc(static_cast<const char*>(m.scales) + (size_t)e * N * srow, (uint32_t)N * srow);
  d.b = make_rsrc(static_cast<const char*>(m.biases) + (size_t)e * N * srow, (uint32_t)N * srow);
  return d;
}

// Row n for lane column ll (at most 2048 wide: 16 scale dwords).
template <int C>
__device__ __forceinline__ void ds_load_row(const DsMat& m, int n, int kin, int ll, DsRow<C>& w) {
  static_assert(C <= 4, "rows of at most 2048 elements");
  const uint32_t qrow = (uint32_t)kin * kBits / 8, srow = (uint32_t)kin / 32;
  const uint32_t so = (uint32_t)n * srow + 4u * (4u * (ll & 3) + (ll >> 2));
  w.s = __builtin_amdgcn_raw_buffer_load_b32(m.s, so, 0, 0);
  w.b = __builtin_amdgcn_raw_buffer_load_b32(m.b, so, 0, 0);
#pragma unroll
  for (int c = 0; c < C; ++c) {
    const uint32_t qo = (uint32_t)n * qrow + 16u * kQW * (16u * c + ll);
#pragma unroll
    for (int j = 0; j < kQW; ++j)
      w.q[c][j] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(m.q, qo + 16u * j, 0, 0));
  }
}

// Lane 4 (lane / 4) + c's value in every lane of its quad (DPP quad_perm).
__device__ __forceinline__ uint32_t quad_bcast(uint32_t v, int c) {
  switch (c & 3) {
    case 0: return __builtin_amdgcn_mov_dpp(v, 0x00, 0xf, 0xf, false);
    case 1: return __builtin_amdgcn_mov_dpp(v, 0x55, 0xf, 0xf, false);
    case 2: return __builtin_amdgcn_mov_dpp(v, 0xaa, 0xf, 0xf, false);
    default: return __builtin_amdgcn_mov_dpp(v, 0xff, 0xf, 0xf, false);
  }
}

// Scale or bias of chunk c (group 8c + ll / 2) from a row's dword (DsRow):
// the high half of the broadcast dword for ll % 4 in {2, 3}.
__device__ __forceinline__ float ds_row_sb(uint32_t v, int c, int ll) {
  const uint32_t d = quad_bcast(v, c);
  if constexpr (kF16) {
    return st2f<true>((uint16_t)__builtin_amdgcn_perm(0u, d, (ll & 2) ? 0x0c0c0302u : 0x0c0c0100u));
  } else {
    return __uint_as_float(__builtin_amdgcn_perm(0u, d, (ll & 2) ? 0x03020c0cu : 0x01000c0cu));
  }
}

constexpr int kDsXChunks = 4;  // most x chunks staged per thread by the gate/up prologue

// Store one raw 32-element x chunk (4 x 16 bytes) in dot2 pair order:
// xs[(slot*4 + q)*nch + k], and its sum in xsum[slot*nch + k].
__device__ __forceinline__ void ds_store_chunk(const uint4 (&r)[4], uint4* xs, float* xsum, int slot, int k,
                                               int nch) {
  const uint32_t ones = ones2(kF16);  // (1.0, 1.0) in the storage dtype
  float sum = 0.0f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint4 v = r[i];
    xs[(slot * 4 + i) * nch + k] = make_uint4(__builtin_amdgcn_perm(v.y, v.x, 0x05040100u),
                                              __builtin_amdgcn_perm(v.w, v.z, 0x05040100u),
                                              __builtin_amdgcn_perm(v.y, v.x, 0x07060302u),
                                              __builtin_amdgcn_perm(v.w, v.z, 0x07060302u));
    sum = dot2_st<kF16>(v.x, ones, sum);
    sum = dot2_st<kF16>(v.y, ones, sum);
    sum = dot2_st<kF16>(v.z, ones, sum);
    sum = dot2_st<kF16>(v.w, ones, sum);
  }
  xsum[slot * nch + k] = sum;
}

// Stage one 32-element x chunk in pair order: xs[(slot*4 + q)*nch + k], xsum[slot*nch + k].
__device__ __forceinline__ void ds_stage_chunk(const uint16_t* __restrict__ src, uint4* xs, float* xsum,
                                               int slot, int k, int nch) {
  ChunkX cx;
  load_x<kF16>(src, cx);
#pragma unroll
  for (int q = 0; q < 4; ++q)
    xs[(slot * 4 + q) * nch + k] = make_uint4(cx.p[4 * q], cx.p[4 * q + 1], cx.p[4 * q + 2], cx.p[4 * q + 3]);
  xsum[slot * nch + k] = cx.sum;
}

// ---------------------------------------------------------------------------
// 3. gate/up GEMV + SwiGLU: h[j, n] = bf16(silu(x_t . gate_n) * (x_t . up_n)),
// t = order[j] / K, for sorted routes j. Item = 4 rows of gate and of up. Two
// items are in flight per wave: the loads of item i+2 go out as soon as the
// dot products of item i have consumed its registers.
struct DsGateUpArgs {
  const uint16_t* x;       // [T, H]
  const uint16_t* logits;  // [T, E] (ranked modes)
  int32_t* idx;            // [T*K] flat route ids: written (ranked) or read (given)
  float* gates;            // [T*K] flat fp32 gates: written (ranked) or read (given)
  int T, K, E, H, I;
  tfm_affine gate, up;
  Grouping grp;            // published by workgroup 0, with slots and gates_sorted
  uint32_t* status;
  uint16_t* h;  // [R, I]
  // Down weights to prefetch for ds_down_combine_kernel (q null: none, the
  // default; the caller passes them only on request). Its workgroup b reads
  // rows 4b..4b+3 of every routed expert.
  tfm_affine pf;
};

// 16 bytes per lane into LDS at dst + 16 * lane; out-of-range offsets read zero.
__device__ __forceinline__ void ds_lds_copy16(__amdgpu_buffer_rsrc_t r, uint4* dst, uint32_t voff) {
#if defined(__HIP_DEVICE_COMPILE__)
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)dst, 16, voff, 0, 0, 0);
#else
  (void)r; (void)dst; (void)voff;
#endif
}

// Codes of x group q of a chunk (elements 8q..8q+7, staged as the pairs
// (0,2) (4,6) (1,3) (5,7) in v) dotted with v: d += sum x (base + code)
// (4-bit); d += sum x (base + lo), dh += sum x (base + hi) (8-bit).
__device__ __forceinline__ void ds_word_dot(const uint4 (&r)[kQW], int q, const uint4& v, float& d, float& dh) {
  if constexpr (kBits == 4) {
    // Opaque copy: keeps the unpack inside the route loop (hoisted out of
    // it, the unpacked item would need many more registers).
    uint32_t wq = word_of(r[0], q);
    asm volatile("" : "+v"(wq));
    uint32_t p[4];
    unpack_word_st<kF16>(wq, p);
    d = dot2_st<kF16>(p[0], v.x, d);
    d = dot2_st<kF16>(p[1], v.y, d);
    d = dot2_st<kF16>(p[2], v.z, d);
    d = dot2_st<kF16>(p[3], v.w, d);
    (void)dh;
  } else {
    // Words 2q and 2q+1 of the chunk hold codes 8q..8q+3 and 8q+4..8q+7.
    uint32_t wa = word_of(r[q >> 1], (2 * q) & 3), wb = word_of(r[q >> 1], (2 * q + 1) & 3);
    asm volatile("" : "+v"(wa), "+v"(wb));
    const uint32_t magic = kF16 ? 0x64646464u : 0x43434343u;
    const uint32_t la = wa & 0x0f0f0f0fu, ha = (wa >> 4) & 0x0f0f0f0fu;
    const uint32_t lb = wb & 0x0f0f0f0fu, hb = (wb >> 4) & 0x0f0f0f0fu;
    d = dot2_st<kF16>(__builtin_amdgcn_perm(magic, la, 0x04020400u), v.x, d);   // codes 0, 2
    d = dot2_st<kF16>(__builtin_amdgcn_perm(magic, lb, 0x04020400u), v.y, d);   // codes 4, 6
    d = dot2_st<kF16>(__builtin_amdgcn_perm(magic, la, 0x04030401u), v.z, d);   // codes 1, 3
    d = dot2_st<kF16>(__builtin_amdgcn_perm(magic, lb, 0x04030401u), v.w, d);   // codes 5, 7
    dh = dot2_st<kF16>(__builtin_amdgcn_perm(magic, ha, 0x04020400u), v.x, dh);
    dh = dot2_st<kF16>(__builtin_amdgcn_perm(magic, hb, 0x04020400u), v.y, dh);
    dh = dot2_st<kF16>(__builtin_amdgcn_perm(magic, ha, 0x04030401u), v.z, dh);
    dh = dot2_st<kF16>(__builtin_amdgcn_perm(magic, hb, 0x04030401u), v.w, dh);
  }
}

// s * sum x w over one chunk from its code dots: fma(s, d [+ 16 dh], c * sum x).
__device__ __forceinline__ float ds_chunk_value(float s, float d, float dh, float cxs) {
  if constexpr (kBits == 4)
    return __builtin_fmaf(s, d, cxs);
  else
    return __builtin_fmaf(s, __builtin_fmaf(16.0f, dh, d), cxs);
}

template <int C>
struct DsGU {
  DsRow<C> g, u;
};

// Dot products of one gate/up item with one staged token row:
// ag/au = sum over the lane's chunks of s*sum(x(128+q)) + (b-128s)*sum(x).
// The four LDS reads of a chunk go out together, ahead of its dot products.
template <int C>
__device__ __forceinline__ void ds_gu_dot(const DsGU<C>& w, const uint4* __restrict__ xs,
                                          const float* __restrict__ xsum, int tok, int ll, float& ag,
                                          float& au) {
  constexpr int nch = 16 * C;
  ag = au = 0.0f;
#pragma unroll
  for (int c = 0; c < C; ++c) {
    const int k = 16 * c + ll;
    uint4 v[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) v[q] = xs[(tok * 4 + q) * nch + k];
    const float xsm = xsum[tok * nch + k];
    const float sg = ds_row_sb(w.g.s, c, ll), su = ds_row_sb(w.u.s, c, ll);
    const float cg = __builtin_fmaf(-code_corr(), sg, ds_row_sb(w.g.b, c, ll));
    const float cu = __builtin_fmaf(-code_corr(), su, ds_row_sb(w.u.b, c, ll));
    float dg = 0.0f, du = 0.0f, dgh = 0.0f, duh = 0.0f;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      ds_word_dot(w.g.q[c], q, v[q], dg, dgh);
      ds_word_dot(w.u.q[c], q, v[q], du, duh);
    }
    ag += ds_chunk_value(sg, dg, dgh, cg * xsm);
    au += ds_chunk_value(su, du, duh, cu * xsm);
  }
}

// CW = 1 adds one copy wave to the NT compute threads (workgroup NT + 64):
// it routes like the others and then issues every down-weight copy of its
// workgroup, so the compute waves' code holds no copy and their LDS reads
// never wait for one.
template <int C, int XCH, int NT, int PIPE, int MODE, int CW>
__global__ __launch_bounds__(NT + 64 * CW) void ds_gateup_kernel(DsGateUpArgs A) {
  extern __shared__ uint4 ds_lds[];
  const int H = A.H, N = A.I, T = A.T, K = A.K, E = A.E;
  const int R = T * K;
  constexpr int nch = 16 * C;
  // Dynamic LDS: the grouping's scratch, later overwritten by the staged x
  // rows, then the route tokens (ds_gateup_lds sizes it).
  DsGroupLds& GL = *reinterpret_cast<DsGroupLds*>(ds_lds);
  uint4* xs = ds_lds;                                        // [T][4][nch]
  float* xsum = reinterpret_cast<float*>(xs + T * 4 * nch);  // [T][nch]
  const int xbytes = T * nch * 68;
  int* s_tok = reinterpret_cast<int*>(reinterpret_cast<char*>(ds_lds) +
                                      (xbytes > (int)sizeof(DsGroupLds) ? xbytes : (int)sizeof(DsGroupLds)));
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int ll = lane & 15, rsub = lane >> 4;
  const int gw = blockIdx.x * (NT / 64) + (tid >> 6), nw = gridDim.x * (NT / 64);
  // The copy wave (CW = 1): its thread ids start at NT, past every x chunk
  // (XCH = 1 and T * nch <= NT), the routes and the route tokens.
  const bool copier = CW != 0 && (tid >> 6) == NT / 64;

  // Prologue. The x rows of every token (at most XCH 32-element chunks per
  // thread) are requested first; every workgroup then routes and groups the
  // T*K routes itself (a few hundred VALU operations, cheaper than one more
  // dependent kernel launch) and workgroup 0 publishes the result for the
  // down projection and the combine. The first items' weights go out as soon
  // as the grouping is known.
  uint4 xr[XCH][4];
#pragma unroll
  for (int u = 0; u < XCH; ++u) {
    const int p = tid + NT * u;
    if (p < T * nch) {
      const uint4* src = reinterpret_cast<const uint4*>(A.x + (int64_t)(p / nch) * H + 32 * (p % nch));
#pragma unroll
      for (int v = 0; v < 4; ++v) xr[u][v] = src[v];
    }
  }
  auto stage_x = [&]() {
#pragma unroll
    for (int u = 0; u < XCH; ++u) {
      const int p = tid + NT * u;
      if (p < T * nch) ds_store_chunk(xr[u], xs, xsum, p / nch, p % nch, nch);
    }
  };
  // One token with ranked routes: its K routes go to K distinct experts, so
  // the grouping is the ascending order of the chosen ids (sorted position of
  // route f = chosen ids below its own). Every wave routes the token itself,
  // which needs no LDS and no barrier before its first weight loads, and the
  // x row is staged before any weight load is issued, so that waiting for it
  // does not wait for those loads.
  const bool one = MODE != kDsGiven && T == 1;
  // Two to four tokens with ranked routes (at most 64 routes): wave t < T
  // ranks token t and hands its chosen-id mask to the others through LDS;
  // after one barrier every wave reads the grouping off the T masks. Route
  // (t, k) to expert e sits at sorted position off(e) + (tokens before t that
  // chose e), off(e) = the routes of all tokens to experts below e. No
  // grouping scratch, so the x rows are staged before that barrier.
  const bool few = MODE != kDsGiven && T >= 2 && T <= 4 && T <= NT / 64 && R <= 64;
  const int wave = uni(tid >> 6);
  __shared__ uint64_t s_fmask[4];
  __shared__ int s_fid[64];
  uint64_t fm0 = 0, fm1 = 0, fm2 = 0, fm3 = 0;  // few tokens: chosen-id masks of tokens 0-3
  int off_e = 0;                                 // few tokens: routes to experts below lane e
  const bool hro = ds_h_route_order(MODE, T, K);  // h rows in route order
  int pf_e = -1;  // route f's expert in lane f, for the down-weight prefetch
  int4 sl = make_int4(-1, 0, 0, 0);
  uint64_t chosen = 0;          // one token: mask of the chosen ids
  float gv = 0.0f;              // one or few tokens: lane f's (lane k's) gate
  int id = -1, pos = 0, ex = -1;  // one or few tokens: the route's id and sorted position; lane a's expert
  int ordv = 0;                   // one token: lane a's route
  if (one) {
    if (MODE == TFM_ROUTE_OLMOE) {
      uint16_t gb;
      id = olmoe_route_wave<kF16>(A.logits, E, K, &gv, &gb, &chosen);
    } else {
      id = granite_route_wave<kF16>(A.logits, E, K, &gv, &chosen);
    }
    const bool route = lane < K;
    pos = route ? __popcll(chosen & ((1ull << id) - 1ull)) : lane;
    // Lane a < K receives the expert and the route at sorted position a.
    ex = __builtin_amdgcn_ds_permute(4 * pos, route ? id : -1);
    ordv = __builtin_amdgcn_ds_permute(4 * pos, lane);
    sl = lane < K ? make_int4(ex, lane, lane + 1, K) : make_int4(-1, 0, 0, K);
    if (A.pf.q != nullptr && route) pf_e = id;
    stage_x();
  } else if (few) {
    if (wave < T) {
      uint64_t ch = 0;
      if (MODE == TFM_ROUTE_OLMOE) {
        uint16_t gb;
        id = olmoe_route_wave<kF16>(A.logits + (int64_t)wave * E, E, K, &gv, &gb, &ch);
      } else {
        id = granite_route_wave<kF16>(A.logits + (int64_t)wave * E, E, K, &gv, &ch);
      }
      if (lane == 0) s_fmask[wave] = ch;
      if (lane < K) s_fid[wave * K + lane] = id;
    }
    stage_x();
    __syncthreads();  // masks, route ids and x rows visible
    auto uni64 = [](uint64_t v) {
      return (uint64_t)(uint32_t)uni((int)(uint32_t)v) | ((uint64_t)(uint32_t)uni((int)(v >> 32)) << 32);
    };
    fm0 = uni64(s_fmask[0]);
    fm1 = uni64(s_fmask[1]);
    fm2 = T > 2 ? uni64(s_fmask[2]) : 0ull;
    fm3 = T > 3 ? uni64(s_fmask[3]) : 0ull;
    const uint64_t um = fm0 | fm1 | fm2 | fm3;
    const int U = __popcll(um);
    const uint64_t below = lane == 0 ? 0ull : (~0ull >> (64 - lane));
    off_e = __popcll(fm0 & below) + __popcll(fm1 & below) + __popcll(fm2 & below) + __popcll(fm3 & below);
    const int cnt_e = (int)((fm0 >> lane) & 1) + (int)((fm1 >> lane) & 1) + (int)((fm2 >> lane) & 1) +
                      (int)((fm3 >> lane) & 1);
    // Lane e of the union goes to slot a = union ids below e; the other lanes
    // to the slots past U, so that the permute's targets are distinct.
    const bool in = (um >> lane) & 1;
    const int a = __popcll(um & below);
    const int dst = 4 * (in ? a : U + (lane - a));
    ex = __builtin_amdgcn_ds_permute(dst, in ? lane : -1);
    const int j0a = __builtin_amdgcn_ds_permute(dst, off_e);
    const int j1a = __builtin_amdgcn_ds_permute(dst, off_e + cnt_e);
    sl = lane < U ? make_int4(ex, j0a, j1a, U) : make_int4(-1, 0, 0, U);
    if (A.pf.q != nullptr && lane < R) pf_e = s_fid[lane];
    if (wave < T && lane < K) {
      const uint64_t bl = (1ull << id) - 1ull;
      pos = __popcll(fm0 & bl) + __popcll(fm1 & bl) + __popcll(fm2 & bl) + __popcll(fm3 & bl) +
            (wave > 0 ? (int)((fm0 >> id) & 1) : 0) + (wave > 1 ? (int)((fm1 >> id) & 1) : 0) +
            (wave > 2 ? (int)((fm2 >> id) & 1) : 0);
    }
  } else {
    ds_rank_group<MODE>(GL, A.logits, T, E, K, A.idx, A.gates, blockIdx.x == 0, A.grp, A.status);
    __syncthreads();
    // Down-weight prefetch (few tokens): the routes' experts, read before the
    // grouping scratch is overwritten.
    if (A.pf.q != nullptr && lane < R) pf_e = GL.e[lane];
    const int U = GL.act[E];
    if (lane < U) {
      const int ex = GL.act[lane];
      sl = make_int4(ex, GL.off[ex], GL.off[ex + 1], U);
    } else {
      sl.w = U;
    }
  }
  WaveRange wr{};
  const int ipe = (N + 3) / 4;
  if (!copier) wave_range(sl, ipe, gw, nw, wr);
  auto load = [&](DsGU<C>& w, int i) {
    const int a = i / ipe;
    const int e = uni(readlane_i(wr.sl.x, a));
    const int n = (i - a * ipe) * 4 + rsub;
    ds_load_row<C>(ds_mat(A.gate, e, N, H), n, H, ll, w.g);
    ds_load_row<C>(ds_mat(A.up, e, N, H), n, H, ll, w.u);
  };

  // Down-weight prefetch (only when the caller asks for it: reading the down
  // weights from HBM in the down kernel measured faster once that kernel
  // issued its loads right after the route ids). When the down projection runs as
  // ds_down_combine_kernel, its workgroup b' reads rows 4b'..4b'+3 of every
  // routed expert's down matrix: packed codes, scales and biases, three
  // contiguous runs. Workgroup b of this kernel copies them for b' = b,
  // b + grid, ... into a landing area that is never read. The XCDs' L2
  // caches are invalidated between kernels, but the copies stay in the
  // Infinity Cache, which serves the down kernel's loads faster than HBM.
  // Wave w copies routes w, w + NT/64, ... The compiler cannot tell the
  // landing area from the staged x rows, so an LDS read issued after a copy
  // waits for every load in flight: at one token the copies go out after the
  // items (the weight stream bounds this kernel either way).
  __shared__ __attribute__((aligned(16))) uint4 s_sink[NT / 64][64];
  auto prefetch = [&]() {
    if (A.pf.q == nullptr) return;
    const int nb = (A.H + 3) / 4, wave = uni(tid >> 6);
    const int f0 = CW ? 0 : wave, fs = CW ? 1 : NT / 64;  // the copy wave takes every route
    uint4* sink = s_sink[CW ? 0 : wave];
    const uint32_t qrow = (uint32_t)A.I * kBits / 8, srow = (uint32_t)A.I / 32;
    for (int bp = blockIdx.x; bp < nb; bp += gridDim.x) {
      for (int f = f0; f < R; f += fs) {
        const int e = uni(readlane_i(pf_e, f));
        if (e < 0 || e >= E) continue;
        const DsMat m = ds_mat(A.pf, e, A.H, A.I);
        const uint32_t q0 = 4u * bp * qrow, s0 = 4u * bp * srow;
        for (uint32_t o = 0; o < 4 * qrow; o += 1024) ds_lds_copy16(m.q, sink, q0 + o + 16u * lane);
        const uint32_t so = 16u * lane < 4 * srow ? s0 + 16u * lane : 0x80000000u;
        ds_lds_copy16(m.s, sink, so);
        ds_lds_copy16(m.b, sink, so);
      }
    }
  };

  DsGU<C> wA, wB;
  if (one) {
    if (wr.i0 < wr.i1) load(wA, wr.i0);
    if (PIPE == 2 && wr.i0 + 1 < wr.i1) load(wB, wr.i0 + 1);
    asm volatile("; one-token barrier" ::: "memory");
    __syncthreads();  // the x row is staged
    // Published after the barrier: a barrier waits for the global stores in
    // flight, and stores count in the same in-order counter as loads.
    if (blockIdx.x == 0 && tid < 64) {
      if (lane < K) {
        A.idx[lane] = id;
        A.gates[lane] = gv;
        A.grp.order[pos] = lane;
        A.grp.inverse[lane] = pos;
        A.grp.gates_sorted[pos] = gv;
        A.grp.active[lane] = ex;
      }
      if (lane < E) {
        A.grp.offsets[lane] = __popcll(chosen & ((1ull << lane) - 1ull));
        A.grp.slots[lane] = sl;
      }
      if (lane == 0) {
        A.grp.offsets[E] = K;
        A.grp.active[E] = K;
      }
    }
  } else if (few) {
    if (wr.i0 < wr.i1) load(wA, wr.i0);
    if (PIPE == 2 && wr.i0 + 1 < wr.i1) load(wB, wr.i0 + 1);
    // The grouping, published as ds_rank_group publishes it.
    if (blockIdx.x == 0) {
      if (wave < T && lane < K) {
        const int f = wave * K + lane;
        A.idx[f] = id;
        A.gates[f] = gv;
        A.grp.order[pos] = f;
        A.grp.inverse[f] = pos;
        A.grp.gates_sorted[pos] = gv;
      }
      if (wave == 0) {
        const int U = sl.w;
        if (lane < E) {
          A.grp.offsets[lane] = off_e;
          A.grp.slots[lane] = sl;
        }
        if (lane < U) A.grp.active[lane] = ex;
        if (lane == 0) {
          A.grp.offsets[E] = R;
          A.grp.active[E] = U;
        }
      }
    }
    if (!CW) prefetch();
  } else {
    if (wr.i0 < wr.i1) load(wA, wr.i0);
    if (PIPE == 2 && wr.i0 + 1 < wr.i1) load(wB, wr.i0 + 1);
    for (int j = tid; j < R; j += NT) s_tok[j] = GL.order[j] / K;
    __syncthreads();  // the grouping scratch is read; the x rows may overwrite it
    stage_x();
    __syncthreads();
    if (!CW) prefetch();
  }

  auto emit = [&](int j, int n, float ag, float au) {
    const float gt = dpp_group_sum<16>(ag);
    const float up = dpp_group_sum<16>(au);
    if (ll == 0 && n < N) {
      const float hv = gt * __builtin_amdgcn_rcpf(1.0f + __expf(-gt)) * up;
      A.h[(int64_t)j * N + n] = f2st<kF16>(hv);
    }
  };
  // Routes one at a time through one branch-free body (the nibble unpack is
  // redone per route: at decode most experts have one or two routes). PIPE
  // items are in flight per wave: when every route of item i is done, its
  // registers are refilled with item i + PIPE.
  auto step = [&](DsGU<C>& w, int i) {
    const int a = i / ipe;
    const int n = (i - a * ipe) * 4 + rsub;
    const int j0 = uni(readlane_i(wr.sl.y, a)), j1 = uni(readlane_i(wr.sl.z, a));
    // One token whose down projection is the fused down + combine kernel:
    // h row = route (ds_h_route_order), the route of slot a (one route per
    // slot); else the sorted position, which the separate down kernel reads.
    // Read once per item: a read per route raised the kernel to 191 registers.
    const int hr0 = hro ? uni(readlane_i(ordv, a)) : j0;
    // Few tokens: slot a's expert, whose routes are in token order.
    const int ea = few ? uni(readlane_i(wr.sl.x, a)) : 0;
    for (int j = j0; j < j1; ++j) {
      float ag, au;
      int tok = 0;
      if (few) {
        // the (j - j0)-th token that chose expert ea
        int r = j - j0;
        const bool c0 = (fm0 >> ea) & 1, c1 = (fm1 >> ea) & 1, c2 = (fm2 >> ea) & 1;
        tok = c0 && r == 0 ? 0 : (r -= c0, c1 && r == 0 ? 1 : (r -= c1, c2 && r == 0 ? 2 : 3));
      } else if (!one) {
        tok = s_tok[j];
      }
      ds_gu_dot<C>(w, xs, xsum, tok, ll, ag, au);
      emit(hr0 + (j - j0), n, ag, au);
    }
    if (i + PIPE < wr.i1) load(w, i + PIPE);
  };
  // The copy wave's copies sit on a branch of their own that joins the
  // compute waves' only at the end, so that no LDS read of theirs follows a
  // copy in program order.
  if (!copier) {
    if (PIPE == 1) {
      for (int i = wr.i0; i < wr.i1; ++i) step(wA, i);
    } else {
      for (int i = wr.i0; i < wr.i1; i += 2) {
        step(wA, i);
        if (i + 1 < wr.i1) step(wB, i + 1);
      }
    }
    if (!CW && one) prefetch();
  } else {
    prefetch();
  }
}

// ---------------------------------------------------------------------------
// 4. down GEMV scaled by the gate: P[j, n] = gate_j * (h_j . down_n) (fp32),
// sorted routes j. Item = 4*RG rows; two items in flight per wave. Each wave
// stages the h rows of up to kDsDownXB routes of its current expert in its
// own LDS region.
struct DsDownArgs {
  const uint16_t* h;  // [R, I] sorted rows
  int E, H, I;
  tfm_affine down;
  const int4* slots;
  const float* gates_sorted;
  float* P;  // [R, H]
};

template <int C, int RG>
struct DsDn {
  DsRow<C> r[RG];
};

// Dot products of one down item with staged h row t.
template <int C, int RG>
__device__ __forceinline__ void ds_dn_dot(const DsDn<C, RG>& w, const uint4* __restrict__ xs,
                                          const float* __restrict__ xsum, int t, int ll,
                                          float (&acc)[RG]) {
  constexpr int nch = 16 * C;
#pragma unroll
  for (int g = 0; g < RG; ++g) acc[g] = 0.0f;
#pragma unroll
  for (int c = 0; c < C; ++c) {
    const int k = 16 * c + ll;
    uint4 v[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) v[q] = xs[(t * 4 + q) * nch + k];
    const float xsm = xsum[t * nch + k];
    float d[RG], dh[RG];
#pragma unroll
    for (int g = 0; g < RG; ++g) d[g] = dh[g] = 0.0f;
#pragma unroll
    for (int q = 0; q < 4; ++q)
#pragma unroll
      for (int g = 0; g < RG; ++g) ds_word_dot(w.r[g].q[c], q, v[q], d[g], dh[g]);
#pragma unroll
    for (int g = 0; g < RG; ++g) {
      // Opaque copies: keep the conversions here, at the dot products. Moved
      // up to the loads, they make a wave wait for one row's scales before it
      // issues the next row's loads.
      uint32_t sr = w.r[g].s, br = w.r[g].b;
      asm volatile("" : "+v"(sr), "+v"(br));
      const float sc = ds_row_sb(sr, c, ll);
      const float cc = __builtin_fmaf(-code_corr(), sc, ds_row_sb(br, c, ll));
      acc[g] += ds_chunk_value(sc, d[g], dh[g], cc * xsm);
    }
  }
}

template <int C, int RG, int NT, int PIPE>
__global__ __launch_bounds__(NT) void ds_down_kernel(DsDownArgs A) {
  extern __shared__ uint4 ds_lds[];
  constexpr int XB = kDsDownXB;
  constexpr int nch = 16 * C;
  const int N = A.H, kin = A.I;
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int ll = lane & 15, rsub = lane >> 4;
  const int gw = blockIdx.x * (NT / 64) + wave, nw = gridDim.x * (NT / 64);
  constexpr int region = XB * 4 * nch + (XB * nch + 3) / 4;  // uint4 per wave
  uint4* xs = ds_lds + wave * region;
  float* xsum = reinterpret_cast<float*>(xs + XB * 4 * nch);

  WaveRange wr;
  const int ipe = (N + 4 * RG - 1) / (4 * RG);
  wave_range(load_slot(A.slots, A.E), ipe, gw, nw, wr);
  auto load = [&](DsDn<C, RG>& w, int i) {
    const int a = i / ipe;
    const int e = uni(readlane_i(wr.sl.x, a));
    const int r = i - a * ipe;
    const DsMat m = ds_mat(A.down, e, N, kin);
#pragma unroll
    for (int g = 0; g < RG; ++g) ds_load_row<C>(m, r * 4 * RG + 4 * g + rsub, kin, ll, w.r[g]);
  };
  DsDn<C, RG> wA, wB;
  if (wr.i0 < wr.i1) load(wA, wr.i0);
  if (PIPE == 2 && wr.i0 + 1 < wr.i1) load(wB, wr.i0 + 1);
  int staged_j = -1;  // first route of the staged batch
  float gv = 0.0f;    // lane t: gate of staged route t

  auto stage = [&](int jb, int nb) {
    if (staged_j == jb) return;
    // The previous batch's reads of this region come first in program
    // order, and LDS operations of one wave complete in order.
    for (int p = lane; p < nb * nch; p += 64) {
      const int t = p / nch, k = p % nch;
      ds_stage_chunk(A.h + (int64_t)(jb + t) * kin + 32 * k, xs, xsum, t, k, nch);
    }
    gv = lane < nb ? A.gates_sorted[jb + lane] : 0.0f;
    staged_j = jb;
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  };
  auto emit = [&](int j, int t, int r, const float (&acc)[RG]) {
    const float gt = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(gv), t));
#pragma unroll
    for (int g = 0; g < RG; ++g) {
      const float sum = dpp_group_sum<16>(acc[g]);
      const int n = r * 4 * RG + 4 * g + rsub;
      if (ll == 0 && n < N) A.P[(int64_t)j * N + n] = sum * gt;
    }
  };
  auto step = [&](DsDn<C, RG>& w, int i) {
    const int a = i / ipe;
    const int r = i - a * ipe;
    const int j0 = uni(readlane_i(wr.sl.y, a)), j1 = uni(readlane_i(wr.sl.z, a));
    for (int jb = j0; jb < j1; jb += XB) {
      const int nb = min(XB, j1 - jb);
      stage(jb, nb);
      for (int t = 0; t < nb; ++t) {
        float acc[RG];
        ds_dn_dot<C, RG>(w, xs, xsum, t, ll, acc);
        emit(jb + t, t, r, acc);
      }
    }
    if (i + PIPE < wr.i1) load(w, i + PIPE);
  };
  if (PIPE == 1) {
    for (int i = wr.i0; i < wr.i1; ++i) step(wA, i);
  } else {
    for (int i = wr.i0; i < wr.i1; i += 2) {
      step(wA, i);
      if (i + 1 < wr.i1) step(wB, i + 1);
    }
  }
}

// ---------------------------------------------------------------------------
// Small batches (T <= kDsSmallT): the down GEMV fused with the combine.

// 4+5 for few tokens: y[t, n] = bf16(fma(rm, sum_k gate_{t,k} * (h_{t,k} . down_n), res[t, n]))
// with the products and the k-ordered sum rounded exactly as ds_down_kernel
// followed by combine_sorted_kernel round them. A workgroup owns a block of
// 4 output rows: it stages the h rows of every route in LDS, wave w computes
// the rows' products for routes w, w+4, .. (streaming the rows' weights of
// each routed expert), and wave 0 sums each token's K products in k order.
struct DsDownCombineArgs {
  const uint16_t* h;        // [R, I]: route order (h_route_order) or sorted rows
  int h_route_order;
  const int32_t* idx;       // [R] flat route -> expert
  const float* gates;       // [R] flat route gates
  const int32_t* inverse;   // [R] flat route -> sorted position
  int T, K, E, H, I;
  tfm_affine down;
  const uint16_t* residual;  // [T, H] or null
  float rmul;
  uint16_t* y;  // [T, H]
};

// NT threads: NT/64 waves share the routes (route f to wave f mod NT/64).
// Instances: at most TMAX tokens and RMAX routes, FW = RMAX / (NT/64) routes
// per wave. Batches of up to 2 tokens and 16 routes run the instance sized
// for them: the one sized for 3 tokens made the one-token layer 5% slower.
template <int C, int NT, int RMAX, int TMAX>
__global__ __launch_bounds__(NT) void ds_down_combine_kernel(DsDownCombineArgs A) {
  extern __shared__ uint4 ds_lds[];
  __shared__ float s_p[RMAX][4];  // product of route f for row 4*blockIdx.x + r
  constexpr int nch = 16 * C;
  constexpr int NW = NT / 64;
  constexpr int FW = (RMAX + NW - 1) / NW;  // routes per wave
  static_assert(RMAX <= kDsSmallR && TMAX <= kDsSmallT, "within the small-batch limits");
  const int T = A.T, K = A.K, E = A.E, N = A.H, kin = A.I;
  const int R = T * K;
  uint4* xs = ds_lds;                                        // [R][4][nch]
  float* xsum = reinterpret_cast<float*>(xs + R * 4 * nch);  // [R][nch]
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int ll = lane & 15, rsub = lane >> 4;
  const int n = blockIdx.x * 4 + rsub;
  int fe = -1, fpos = 0;
  float fg = 0.0f;
  if (lane < R) {
    fe = A.idx[lane];
    fg = A.gates[lane];
    fpos = A.inverse[lane];
  }
  // h rows in route order (one token) need no position: their chunks are
  // requested right after the route ids (which the weight loads wait for), at
  // most kDsDcHold per thread, and staged after the
  // weight loads are issued.
  constexpr int kDsDcHold = 2;
  const bool hold = A.h_route_order && R * nch <= kDsDcHold * NT;
  uint4 hr[kDsDcHold][4];
  if (hold) {
#pragma unroll
    for (int u = 0; u < kDsDcHold; ++u) {
      const int p = tid + NT * u;
      if (p < R * nch) {
        const uint4* src = reinterpret_cast<const uint4*>(A.h + (int64_t)(p / nch) * kin + 32 * (p % nch));
#pragma unroll
        for (int v = 0; v < 4; ++v) hr[u][v] = src[v];
      }
    }
  }
  // The residual of this lane's output row for both tokens, requested now so
  // that the final sum does not wait for it.
  // Kept as storage bits until the sum: converted here, they would make the
  // wave wait for every load issued so far.
  uint32_t res[TMAX] = {};
  if (wave == 0 && ll == 0 && n < N && A.residual) {
#pragma unroll
    for (int t = 0; t < TMAX; ++t)
      if (t < T) res[t] = A.residual[(int64_t)t * N + n];
  }
  // This wave's routes' weight rows, then every route's h row (sorted
  // position inverse[f]) into slot f. Bad routes' h rows were never written:
  // they are staged but not used.
  DsDn<C, 1> wt[FW];
#pragma unroll
  for (int u = 0; u < FW; ++u) {
    const int f = wave + NW * u;
    const int e = uni(readlane_i(fe, min(f, R - 1)));
    if (f < R && e >= 0 && e < E) ds_load_row<C>(ds_mat(A.down, e, N, kin), n, kin, ll, wt[u].r[0]);
  }
  if (hold) {
#pragma unroll
    for (int u = 0; u < kDsDcHold; ++u) {
      const int p = tid + NT * u;
      if (p < R * nch) ds_store_chunk(hr[u], xs, xsum, p / nch, p % nch, nch);
    }
  } else {
    for (int p = tid; p < R * nch; p += NT) {
      const int f = p / nch, k = p % nch;
      const int pos = A.h_route_order ? f : __shfl(fpos, f, 64);
      ds_stage_chunk(A.h + (int64_t)pos * kin + 32 * k, xs, xsum, f, k, nch);
    }
  }
  __syncthreads();
#pragma unroll
  for (int u = 0; u < FW; ++u) {
    const int f = wave + NW * u;
    if (f >= R) break;
    const int e = uni(readlane_i(fe, f));
    float pr = 0.0f;
    if (e >= 0 && e < E) {
      float acc[1];
      ds_dn_dot<C, 1>(wt[u], xs, xsum, f, ll, acc);
      const float sum = dpp_group_sum<16>(acc[0]);
      const float gt = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(fg), f));
      pr = __fmul_rn(sum, gt);
    }
    if (ll == 0) s_p[f][rsub] = pr;
  }
  __syncthreads();
  if (wave == 0) {
#pragma unroll
    for (int t = 0; t < TMAX; ++t) {
      if (t >= T) break;
      // Bad routes hold a product of +0, and the sum (from +0) is never -0,
      // so adding them changes no bit: the K reads go out together.
      float sacc = 0.0f;
      for (int k = 0; k < K; ++k) sacc = __fadd_rn(sacc, s_p[t * K + k][rsub]);
      if (ll == 0 && n < N)
        A.y[(int64_t)t * N + n] =
            (uint16_t)pack_st2<kF16>(__builtin_fmaf(A.rmul, sacc, st2f<kF16>((uint16_t)res[t])), 0.0f);
    }
  }
}

// ---------------------------------------------------------------------------
// Host side.

static int device_cus() {
  static int cus = [] {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return 256;
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
      return 256;
    return n;
  }();
  return cus;
}

static int env_int(const char* name, int dflt, int lo, int hi) {
  const char* s = std::getenv(name);
  if (!s) return dflt;
  char* end = nullptr;
  const long v = std::strtol(s, &end, 10);
  if (!end || *end != 0 || v < lo || v > hi) return dflt;
  return (int)v;
}

static size_t ds_gateup_lds(int T, int K, int H) {
  const size_t x = (size_t)T * (H / 32) * 68;  // staged x rows and their chunk sums
  return std::max(x, sizeof(DsGroupLds)) + (size_t)T * K * 4;
}

static size_t ds_down_lds(int I, int threads) {
  const int nch = I / 32;
  return (size_t)(threads / 64) * ((size_t)kDsDownXB * 4 * nch * 16 + (((size_t)kDsDownXB * nch + 3) / 4) * 16);
}

bool decode_stream_fits(int T, int K, int E, int H, int I) {
  const bool w_ok = (H % 512 == 0) && H >= 512 && H <= 2048 && (I % 512 == 0) && I >= 512 && I <= 2048;
  return w_ok && E <= 64 && T * K <= 256 && T >= 1 && T * (H / 32) <= 256 * kDsXChunks &&
         ds_gateup_lds(T, K, H) <= 64 * 1024 &&
         ds_down_lds(I, 256) <= 64 * 1024;
}

// Workgroups resident per compute unit for a kernel at a block and dynamic
// LDS size (cached per kernel and size; the first query goes to the runtime).
template <typename Kern>
static int resident_per_cu(Kern kern, int threads, size_t lds) {
  struct Entry {
    const void* k;
    size_t lds;
    int n;
  };
  static thread_local Entry cache[32];
  static thread_local int used = 0;
  const void* key = reinterpret_cast<const void*>(kern);
  for (int i = 0; i < used; ++i)
    if (cache[i].k == key && cache[i].lds == lds) return cache[i].n;
  int n = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, kern, threads, lds) != hipSuccess || n <= 0) n = 1;
  if (used < 32) cache[used++] = Entry{key, lds, n};
  return n;
}

// One resident round of workgroups (every wave then streams a contiguous
// item range), capped so that every wave has at least one item.
template <typename Kern>
static unsigned ds_grid(Kern kern, int threads, size_t lds, int64_t max_items) {
  const int per_cu = env_int("TFM_DS_WG_PER_CU", resident_per_cu(kern, threads, lds), 1, 16);
  const int64_t cap = (int64_t)device_cus() * per_cu;
  const int64_t want = (max_items + threads / 64 - 1) / (threads / 64);
  return (unsigned)std::max<int64_t>(1, std::min(cap, want));
}

// ds_grid for a gate/up kernel with a copy wave: 320 threads per workgroup,
// of which 4 waves take items.
template <typename Kern>
static unsigned ds_grid_cw(Kern kern, size_t lds, int64_t max_items) {
  const int per_cu = env_int("TFM_DS_WG_PER_CU", resident_per_cu(kern, 320, lds), 1, 16);
  const int64_t cap = (int64_t)device_cus() * per_cu;
  const int64_t want = (max_items + 3) / 4;
  return (unsigned)std::max<int64_t>(1, std::min(cap, want));
}

// Raises a kernel's dynamic LDS limit (64 KiB by default) once per kernel.
template <typename Kern>
static void allow_lds(Kern kern, size_t lds) {
  if (lds <= 64 * 1024) return;
  static thread_local const void* done[16];
  static thread_local int used = 0;
  const void* key = reinterpret_cast<const void*>(kern);
  for (int i = 0; i < used; ++i)
    if (done[i] == key) return;
  check_hip(hipFuncSetAttribute(key, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds),
            "decode down: LDS limit");
  if (used < 16) done[used++] = key;
}

// Threads per workgroup of the streaming GEMVs: 256 measured faster than
// 1024 (one workgroup per compute unit) at decode shapes.
static int ds_threads() {
  const int v = env_int("TFM_DS_THREADS", 256, 256, 1024);
  return v >= 1024 ? 1024 : v >= 512 ? 512 : 256;
}

void launch_ds_gateup(int mode, const uint16_t* x, const uint16_t* logits, int32_t* idx, float* gates,
                      int T, int K, int E, int H, int I, const tfm_affine& gate, const tfm_affine& up,
                      const Grouping& g, uint32_t* status, uint16_t* h, const tfm_affine* pf_down, hipStream_t s) {
  if (T * K > 256 || E > 64) fail(TFM_E_INVALID, "decode gate/up: more than 256 routes or 64 experts");
  DsGateUpArgs A{};
  A.x = x; A.logits = logits; A.idx = idx; A.gates = gates;
  A.T = T; A.K = K; A.E = E; A.H = H; A.I = I; A.gate = gate; A.up = up;
  A.grp = g; A.status = status; A.h = h;
  if (pf_down && decode_small(T, K)) A.pf = *pf_down;
  const size_t lds = ds_gateup_lds(T, K, H);
  const int max_active = T * K < E ? T * K : E;
  const int64_t items = (int64_t)max_active * ((I + 3) / 4);
  const int nt = ds_threads();
  const int pipe = env_int("TFM_DS_PIPE", 1, 1, 2);
  const int per = T * (H / 32);
  const int xch = per <= nt ? 1 : per <= 2 * nt ? 2 : 4;
  // With down-weight copies requested: at one token a copy wave issues them;
  // at two the compute waves do, before their items (TFM_DS_COPY_WAVE=0/1
  // forces either; without the copy wave, one token's copies follow the
  // items). Per layer, copies on: OLMoE 1 token 16.75 us with the copy wave,
  // 17.36 without; 2 tokens 30.8 with, 26.4 without; Granite 2 tokens 17.8
  // either way.
  const bool copy_wave = A.pf.q != nullptr && env_int("TFM_DS_COPY_WAVE", T == 1 ? 1 : 0, 0, 1) == 1;
#define TFM_DS_GU_P(CV, XV, NV, PV, MV)                                                              \
  if (copy_wave && XV == 1 && NV == 256 && PV == 1) {                                              \
    tfm_launch(ds_gateup_kernel<CV, 1, 256, 1, MV, 1>,                                             \
               ds_grid_cw(ds_gateup_kernel<CV, 1, 256, 1, MV, 1>, lds, items), 320, lds, s, A);    \
  } else {                                                                                         \
    tfm_launch(ds_gateup_kernel<CV, XV, NV, PV, MV, 0>,                                            \
               ds_grid(ds_gateup_kernel<CV, XV, NV, PV, MV, 0>, NV, lds, items), NV, lds, s, A);   \
  }
#define TFM_DS_GU_M(CV, XV, NV, PV)                                         \
  if (mode == TFM_ROUTE_OLMOE) { TFM_DS_GU_P(CV, XV, NV, PV, TFM_ROUTE_OLMOE) }     \
  else if (mode == TFM_ROUTE_GRANITE) { TFM_DS_GU_P(CV, XV, NV, PV, TFM_ROUTE_GRANITE) } \
  else { TFM_DS_GU_P(CV, XV, NV, PV, kDsGiven) }
#define TFM_DS_GU_X(CV, XV, NV) \
  if (pipe == 2 && NV == 256) { TFM_DS_GU_M(CV, XV, 256, 2) } else { TFM_DS_GU_M(CV, XV, NV, 1) }
#define TFM_DS_GU(CV)                                           \
  if (nt == 1024) {                                             \
    if (xch == 1) { TFM_DS_GU_X(CV, 1, 1024) } else { TFM_DS_GU_X(CV, 2, 1024) } \
  } else if (nt == 512) {                                       \
    if (xch == 1) { TFM_DS_GU_X(CV, 1, 512) } else { TFM_DS_GU_X(CV, 2, 512) } \
  } else if (xch == 1) { TFM_DS_GU_X(CV, 1, 256) }              \
  else if (xch == 2) { TFM_DS_GU_X(CV, 2, 256) }                \
  else { TFM_DS_GU_X(CV, 4, 256) }
  switch (H / 512) {
    case 1: TFM_DS_GU(1) break;
    case 2: TFM_DS_GU(2) break;
    case 3: TFM_DS_GU(3) break;
    case 4: TFM_DS_GU(4) break;
    default: fail(TFM_E_UNSUPPORTED, "decode gate/up: hidden width");
  }
#undef TFM_DS_GU
#undef TFM_DS_GU_X
#undef TFM_DS_GU_M
#undef TFM_DS_GU_P
  check_hip(hipGetLastError(), "decode gate/up launch");
}

void launch_ds_down(const uint16_t* hsorted, int H, int I, int max_active, const tfm_affine& down,
                    const Grouping& g, float* P, hipStream_t s) {
  DsDownArgs A{};
  A.h = hsorted; A.E = g.E; A.H = H; A.I = I; A.down = down; A.slots = g.slots;
  A.gates_sorted = g.gates_sorted; A.P = P;
  const int nt = ds_down_lds(I, 1024) <= 160 * 1024 - 4096 ? ds_threads() : 256;
  const int pipe = env_int("TFM_DS_PIPE", 1, 1, 2);
  // Rows per item at 512- and 1024-wide h rows (TFM_DS_DOWN_RG = 1, 2 or 4
  // overrides): items of 2-4 KB of packed rows measured fastest, so 8 rows
  // (4-bit codes; 8-bit at 512 wide) or 4 rows (8-bit at 1024 wide). Granite
  // decode (512 wide) at 8 tokens: 36.3 us per layer with 16 rows, 34.8 with
  // 8; 8-bit OLMoE at 8 tokens: 85.4 with 8 rows, 84.0 with 4.
  const int rg = env_int("TFM_DS_DOWN_RG", kBits == 8 && I >= 1024 ? 1 : 2, 1, 4);
  const size_t lds = ds_down_lds(I, nt);
  switch (I / 512) {
#define TFM_DS_DN_P(CV, RV, NV, PV)                                                                      \
  allow_lds(ds_down_kernel<CV, RV, NV, PV>, lds);                                                        \
  tfm_launch(ds_down_kernel<CV, RV, NV, PV>,                                                             \
             ds_grid(ds_down_kernel<CV, RV, NV, PV>, NV, lds, (int64_t)max_active * ((H + 4 * RV - 1) / (4 * RV))), \
             NV, lds, s, A);
#define TFM_DS_DN_N(CV, RV, NV) \
  if (pipe == 2 && NV == 256) { TFM_DS_DN_P(CV, RV, 256, 2) } else { TFM_DS_DN_P(CV, RV, NV, 1) }
#define TFM_DS_DN(CV, RV) \
  if (nt == 1024) { TFM_DS_DN_N(CV, RV, 1024) } else if (nt == 512) { TFM_DS_DN_N(CV, RV, 512) } \
  else { TFM_DS_DN_N(CV, RV, 256) }
    case 1:
      if (rg == 1) {
        TFM_DS_DN(1, 1)
      } else if (rg >= 4) {
        TFM_DS_DN(1, 4)
      } else {
        TFM_DS_DN(1, 2)
      }
      break;
    case 2:
      if (rg == 1) {
        TFM_DS_DN(2, 1)
      } else if (rg >= 4) {
        TFM_DS_DN(2, 4)
      } else {
        TFM_DS_DN(2, 2)
      }
      break;
    case 3: TFM_DS_DN(3, 1) break;
    case 4: TFM_DS_DN(4, 1) break;
#undef TFM_DS_DN
#undef TFM_DS_DN_N
#undef TFM_DS_DN_P
    default: fail(TFM_E_UNSUPPORTED, "decode down: intermediate width");
  }
  check_hip(hipGetLastError(), "decode down launch");
}

void launch_ds_route_group(int route_kind, const uint16_t* logits, int T, int E, int K, int32_t* idx,
                           float* gates, const Grouping& g, uint32_t* status, hipStream_t s) {
  if (T * K > 256 || E > 64 || T <= 0) fail(TFM_E_INVALID, "route+group: more than 256 routes or 64 experts");
  // One wave per token up to 16 waves, at least 4 (the grouping's ballots
  // take 4 waves of 64 routes): fewer waves wait at the grouping's barriers.
  const int nt = 64 * (T < 4 ? 4 : T > 16 ? 16 : T);
  if (route_kind == TFM_ROUTE_OLMOE)
    tfm_launch(ds_route_group_kernel<TFM_ROUTE_OLMOE>, 1, nt, 0, s, logits, T, E, K, idx, gates, g, status);
  else
    tfm_launch(ds_route_group_kernel<TFM_ROUTE_GRANITE>, 1, nt, 0, s, logits, T, E, K, idx, gates, g, status);
  check_hip(hipGetLastError(), "route+group launch");
}

// At most kDsSmallT tokens and kDsSmallR routes (every route's h row is
// staged in LDS, and each route's data sits in one lane).
bool decode_small(int T, int K) { return T >= 1 && T <= kDsSmallT && T * K <= kDsSmallR; }

void launch_ds_down_combine(const uint16_t* h, bool h_route_order, const int32_t* idx, const float* gates,
                            const int32_t* inverse, int T, int K, int E, int H, int I, const tfm_affine& down,
                            const uint16_t* residual, float rmul, uint16_t* y, hipStream_t s) {
  if (!decode_small(T, K)) fail(TFM_E_INVALID, "decode down+combine: batch too large");
  DsDownCombineArgs A{};
  A.h = h; A.h_route_order = h_route_order ? 1 : 0; A.idx = idx; A.gates = gates; A.inverse = inverse;
  A.T = T; A.K = K; A.E = E; A.H = H; A.I = I; A.down = down; A.residual = residual; A.rmul = rmul; A.y = y;
  const int R = T * K;
  const size_t lds = (size_t)R * (I / 32) * 68;
  const unsigned grid = (unsigned)((H + 3) / 4);
  // Eight waves (one route each at one token) unless TFM_DS_DC_THREADS=256.
  const int nt = env_int("TFM_DS_DC_THREADS", 512, 256, 512) >= 512 ? 512 : 256;
  const bool two = T <= 2 && R <= 16;  // the instance for at most 2 tokens and 16 routes
#define TFM_DS_DC_F(CV, NV, RV, TV)                                     \
  {                                                                     \
    allow_lds(ds_down_combine_kernel<CV, NV, RV, TV>, lds);             \
    tfm_launch(ds_down_combine_kernel<CV, NV, RV, TV>, grid, NV, lds, s, A); \
  }
#define TFM_DS_DC(CV)                                                                             \
  if (nt == 512) {                                                                                \
    if (two) TFM_DS_DC_F(CV, 512, 16, 2) else TFM_DS_DC_F(CV, 512, kDsSmallR, kDsSmallT)         \
  } else {                                                                                        \
    if (two) TFM_DS_DC_F(CV, 256, 16, 2) else TFM_DS_DC_F(CV, 256, kDsSmallR, kDsSmallT)         \
  }
  switch (I / 512) {
    case 1: TFM_DS_DC(1) break;
    case 2: TFM_DS_DC(2) break;
    case 3: TFM_DS_DC(3) break;
    case 4: TFM_DS_DC(4) break;
    default: fail(TFM_E_UNSUPPORTED, "decode down+combine: intermediate width");
  }
#undef TFM_DS_DC
#undef TFM_DS_DC_F
  check_hip(hipGetLastError(), "decode down+combine launch");
}

}  // namespace TFM_DS_NS
}  // namespace tfm
