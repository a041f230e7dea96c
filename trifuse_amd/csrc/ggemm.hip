// Prefill path: grouped GEMM over expert-contiguous routes.
//
// Each workgroup computes a BM x BN tile of one expert's output with eight
// waves, two per SIMD, so that one wave's loads, dequantisation and LDS
// traffic overlap the other's MFMAs. Per K step of 64 (one quantisation
// group) it
//   * copies BM activation rows (x rows of the routed tokens, or rows of the
//     expert-sorted SwiGLU output) from global memory straight into LDS
//     (buffer loads with an LDS destination),
//   * loads BN packed weight rows (4-bit: 32 bytes, 8-bit: 64 bytes of each
//     row per step) into registers, dequantises them (s*q+b in fp32,
//     rounded to the storage dtype, bf16 or half) and writes them to LDS;
//     for inputs up to 2048 wide the scales and biases of the tile's rows
//     are copied into LDS once per tile (coalesced) instead of being loaded
//     per step as 2-byte values from 64 rows at a time,
//   * runs v_mfma_f32_32x32x16_bf16 (or _f16) on the two LDS tiles, each wave owning a
//     WM x WN sub-tile (WM*WN/64 fp32 accumulators per lane); 32-row blocks
//     past the end of the expert's segment skip their fragment reads and MFMAs.
//
// Pipeline: two LDS stages for each operand. While the MFMAs of step k read
// stage k%2, the activations of step k+1 are copied into stage (k+1)%2, the
// packed weights of step k+1 (loaded during step k-1) are dequantised into
// stage (k+1)%2 and the packed weights of step k+2 are loaded; one barrier
// per step.
//
// LDS rows are 64 bf16 (8 chunks of 16 B); chunk c of row r is stored at
// c ^ ((r >> 1) & 7), so the 16 lanes of a ds_read_b128 pass (16 consecutive
// rows, one chunk) hit 16 distinct 16-byte bank groups.
//
// Rows outside the segment and weight rows past N get a buffer offset beyond
// the buffer and read as zero, so the loop has no divergent branches.
//
// Epilogue: each wave converts its accumulators (SwiGLU for gate/up) to bf16
// in a private LDS block, 32 rows at a time, and writes them out as 16-byte
// row chunks: h rows (gate/up), expert-output rows in sorted order (down) or
// rows scattered to their flat route (gather_qmm).
#include <cstdlib>
#include <type_traits>

#include "tfm_device.h"
#include "tfm_internal.h"

namespace tfm {

constexpr int BK = 64;
constexpr uint32_t kOob = 0x80000000u;  // buffer offset that reads as zero

enum GgemmMode { kGgGateUp = 0, kGgDown = 1, kGgPlain = 2 };

struct GgArgs {
  const uint16_t* x;     // activations (x rows, or sorted h rows for down)
  uint32_t x_bytes;      // size of x (buffer range)
  RowMap rm;
  Grouping g;
  tfm_affine wa, wb;     // gate/up (wb unused otherwise)
  int N;                 // output columns of one matrix
  int Kin;
  uint16_t* out;         // gate/up: h [n_routes, N]; down: y [n_routes, N]; plain: out [rows, N]
  int sb_layout;         // ggemm_wr_kernel's scale/bias layout in LDS (kSbPlain, kSbDword, kSbChunk)
};

// Scale/bias layouts of ggemm_wr_kernel's LDS copy (see there).
enum { kSbPlain = 0, kSbDword = 1, kSbChunk = 2 };

// Row of accumulator element v of lane `lane` inside a 32x32 block of
// v_mfma_f32_32x32x16_bf16 (its column is lane % 32; operands: lane l
// supplies row/column l%32 and k = 8*(l/32) .. 8*(l/32)+7).
__device__ __forceinline__ int acc_row(int v, int lane) { return 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3); }

__device__ __forceinline__ int swz(int row, int chunk) {
  return row * BK + ((chunk ^ ((row >> 1) & 7)) << 3);
}

__device__ __forceinline__ __amdgpu_buffer_rsrc_t gg_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}

// 4 bytes (one 32-bit word of an 8-bit weight row) -> 4 values s*q+b in the
// storage dtype (bf16, or half when F16).
template <bool F16>
__device__ __forceinline__ uint2 dequant_word_u8(uint32_t w, float s, float b) {
  float d[4];
  dequant4_u8(w, s, b, d);
  uint2 pk;
  pk.x = pack_st2<F16>(d[0], d[1]);
  pk.y = pack_st2<F16>(d[2], d[3]);
  return pk;
}

// 8 nibbles (one 32-bit word of a 4-bit weight row) -> 8 values s*q+b.
template <bool F16>
__device__ __forceinline__ uint4 dequant_word(uint32_t w, float s, float b) {
  float d[8];
  dequant8(w, s, b, d);
  uint4 pk;
  pk.x = pack_st2<F16>(d[0], d[1]);
  pk.y = pack_st2<F16>(d[2], d[3]);
  pk.z = pack_st2<F16>(d[4], d[5]);
  pk.w = pack_st2<F16>(d[6], d[7]);
  return pk;
}

// One 32x32x16 MFMA on bf16 or half operands (fp32 accumulators).
template <bool F16>
using op8_t = std::conditional_t<F16, f16x8_t, bf16x8_t>;
template <bool F16>
__device__ __forceinline__ f32x16_t mfma32(op8_t<F16> a, op8_t<F16> b, f32x16_t c) {
  if constexpr (F16)
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// silu(g) * u with the hardware exp and reciprocal (relative error ~1e-7,
// far below the bf16 rounding that follows).
__device__ __forceinline__ float swiglu(float g, float u) {
  const float e = __builtin_amdgcn_exp2f(-g * 1.44269504f);
  return g * __builtin_amdgcn_rcpf(1.0f + e) * u;
}

// 16 bytes per lane from a buffer into LDS: lane l writes dst + 16*l (dst is
// wave-uniform). Out-of-range offsets deliver zeros.
__device__ __forceinline__ void lds_dma16(__amdgpu_buffer_rsrc_t r, uint16_t* dst, uint32_t voff, uint32_t soff) {
#if defined(__HIP_DEVICE_COMPILE__)
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)dst, 16, voff, soff, 0, 0);
#else
  (void)r; (void)dst; (void)voff; (void)soff;
#endif
}

// The same with 4 bytes per lane: lane l's dword lands at dst + 4 l bytes.
__device__ __forceinline__ void lds_dma4(__amdgpu_buffer_rsrc_t r, uint16_t* dst, uint32_t voff) {
#if defined(__HIP_DEVICE_COMPILE__)
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)dst, 4, voff, 0, 0, 0);
#else
  (void)r; (void)dst; (void)voff;
#endif
}

// Calls f(std::integral_constant<int, I>) for I = B .. E-1 (compile-time
// iteration: every index into register arrays is a constant).
template <int B, int E, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (B < E) {
    f(std::integral_constant<int, B>{});
    static_for<B + 1, E>(f);
  }
}

template <int BM_, int BN_, int WAVES_M_, int WAVES_N_, int MODE, int BITS_>
struct GgCfg {
  static constexpr int BM = BM_, BN = BN_, WAVES_M = WAVES_M_, WAVES_N = WAVES_N_, BITS = BITS_;
  static constexpr int CPR_B = BITS / 2;            // 16-byte packed chunks of a weight row per step
  static constexpr int WAVES = WAVES_M * WAVES_N;
  static constexpr int THREADS = WAVES * 64;
  static constexpr int WM = BM / WAVES_M, WN = BN / WAVES_N;
  static constexpr int MB = WM / 32;                // 32-row MFMA blocks per wave
  static constexpr int NB = WN / 32;                // 32-column MFMA blocks per wave
  static constexpr int LA = BM / (8 * WAVES);       // 8-row LDS copies per wave per step
  static constexpr int LB = BN * CPR_B / THREADS;   // packed 16-byte chunks per thread per step
  static constexpr int OUT_COLS = MODE == kGgGateUp ? BN / 2 : BN;
  static constexpr int WCOLS = MODE == kGgGateUp ? WN / 2 : WN;   // output columns per wave
  static constexpr int SROW = WCOLS + 8;            // staging row stride (bf16), 16 B pad
  static_assert(LA >= 1 && LA * 8 * WAVES == BM, "A copies must tile the block rows");
  static_assert(BITS == 4 || BITS == 8, "4-bit or 8-bit weights");
  static_assert(LB >= 1 && LB * THREADS == BN * CPR_B, "B chunks must tile the block columns");
  static_assert(64 % CPR_B == 0 && (64 / CPR_B) <= BN / 2, "a wave's chunks stay in one half of the tile");
  static_assert(LB * 4 >= 3, "B words are spread over three sub-steps");
  static_assert(MODE != kGgGateUp || NB % 2 == 0, "gate/up wave tiles pair gate and up blocks");
  static_assert(WAVES % 4 == 0, "staging blocks are spread over the four LDS stages");
  static_assert(32 * SROW * (WAVES / 4) <= BM * BK, "epilogue staging must fit in an A stage");
};

// Packed weights of one K step for one thread.
template <int LB>
struct RawB {
  uint4 b[LB];
  uint32_t s[LB], bias[LB];
};

// Largest input width whose scales and biases a tile keeps in LDS (32 groups
// per weight row); wider inputs load them per step with the packed codes.
constexpr int kLdsScaleKin = 32 * BK;

template <int BM_, int BN_, int WAVES_M_, int WAVES_N_, int MODE, int BITS, bool F16, bool SL>
__global__ __launch_bounds__(WAVES_M_ * WAVES_N_ * 64, 1) void ggemm_kernel(GgArgs args) {
  using C = GgCfg<BM_, BN_, WAVES_M_, WAVES_N_, MODE, BITS>;
  constexpr int CPR_B = C::CPR_B;
  constexpr int BM = C::BM, BN = C::BN, MB = C::MB, NB = C::NB, LA = C::LA, LB = C::LB;
  constexpr int T = C::THREADS;
  // Two stages each of A and B, as separate objects so that the compiler's
  // wait tracking tells LDS copies into one stage from reads of the other.
  __shared__ __attribute__((aligned(16))) uint16_t sA0[BM * BK];
  __shared__ __attribute__((aligned(16))) uint16_t sA1[BM * BK];
  __shared__ __attribute__((aligned(16))) uint16_t sB0[BN * BK];
  __shared__ __attribute__((aligned(16))) uint16_t sB1[BN * BK];
  // SL: scales and biases of the tile's weight rows for the whole input
  // width (up to 32 groups per row), copied once per tile.
  __shared__ __attribute__((aligned(16))) uint16_t sSc[SL ? BN * 32 : 8];
  __shared__ __attribute__((aligned(16))) uint16_t sBi[SL ? BN * 32 : 8];
  // The tile prefix and the expert index live in weight stage 1, which is
  // first written after the prologue's barrier.
  int* const s_tiles = reinterpret_cast<int*>(sB1);
  int& s_expert = s_tiles[65];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int E = args.g.E;

  // M-tile prefix over experts.
  if (tid < 64) {
    int t = 0;
    if (tid < E) {
      const int cnt = grp_offset(args.g, tid + 1) - grp_offset(args.g, tid);
      t = (cnt + BM - 1) / BM;
    }
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      const int o = __shfl_up(t, d, 64);
      if (lane >= d) t += o;
    }
    s_tiles[tid + 1] = t;
    if (tid == 0) s_tiles[0] = 0;
  }
  __syncthreads();
  const int NT = (args.N + C::OUT_COLS - 1) / C::OUT_COLS;
  const int mtiles = s_tiles[E];
  const int64_t total = (int64_t)mtiles * NT;
  // XCD-aware remap: workgroups are dispatched round-robin over 8 XCDs, so
  // XCD x gets a contiguous range of tiles (m-tile major) for L2 reuse.
  const int xcd = blockIdx.x & 7;
  const int64_t local = blockIdx.x >> 3;
  const int64_t share = (total + 7) / 8;
  const int64_t ti = xcd * share + local;
  if (local >= share || ti >= total) return;
  const int mt = (int)(ti / NT), nt = (int)(ti % NT);
  if (tid < E && s_tiles[tid] <= mt && mt < s_tiles[tid + 1]) s_expert = tid;
  __syncthreads();
  const int e = s_expert;
  const int seg0 = grp_offset(args.g, e), seg1 = grp_offset(args.g, e + 1);
  const int m0 = seg0 + (mt - s_tiles[e]) * BM;
  const int rows_valid = min(BM, seg1 - m0);
  const int n0 = nt * C::OUT_COLS;
  const int KT = args.Kin / BK;

  // ---- A: global -> LDS copies ----
  // Wave w fills rows [w*BM/W, (w+1)*BM/W), 8 rows (1 KB) per instruction:
  // lane l of copy i writes LDS slot l%8 of row w*BM/W + i*8 + l/8, which
  // under the swizzle holds chunk (l%8) ^ ((row >> 1) & 7).
  const __amdgpu_buffer_rsrc_t ra = gg_rsrc(args.x, args.x_bytes);
  const __amdgpu_buffer_rsrc_t rnull = gg_rsrc(args.x, 0);
  uint32_t a_off[LA];
#pragma unroll
  for (int i = 0; i < LA; ++i) {
    const int r = wave * (BM / C::WAVES) + i * 8 + (lane >> 3);
    const int c = (lane & 7) ^ ((r >> 1) & 7);
    if (r < rows_valid) {
      const int64_t src = MODE == kGgDown ? (int64_t)(m0 + r) : route_row(args.rm, m0 + r);
      a_off[i] = (uint32_t)((src * args.Kin + c * 8) * 2);
    } else {
      a_off[i] = kOob;
    }
  }
  // Step kt of A into LDS stage `dst`; steps past the last read zeros.
  auto a_copy = [&](uint16_t* dst, int kt) {
    const __amdgpu_buffer_rsrc_t r = kt < KT ? ra : rnull;
#pragma unroll
    for (int i = 0; i < LA; ++i) lds_dma16(r, dst + (wave * (BM / C::WAVES) + i * 8) * BK, a_off[i], kt * BK * 2);
  };

  // ---- B: packed weights ----
  // Chunk q = i*T + tid -> weight row q/CPR_B, part q%CPR_B (16 bytes: 32
  // nibbles or 16 bytes of codes). Gate/up tiles hold BN/2 gate rows then
  // BN/2 up rows.
  const uint32_t qrow = (uint32_t)args.Kin * BITS / 8, srow = (uint32_t)(args.Kin / BK) * 2;
  __amdgpu_buffer_rsrc_t rbq[LB], rbs[LB], rbb[LB];
  uint32_t b_qoff[LB], b_soff[LB];
#pragma unroll
  for (int i = 0; i < LB; ++i) {
    const int qw = i * T + wave * 64;  // first chunk of this wave (uniform)
    const bool up = MODE == kGgGateUp && qw / CPR_B >= BN / 2;
    const tfm_affine& bm = up ? args.wb : args.wa;
    const int q = qw + lane;
    const int r = q / CPR_B;
    const int bn = MODE == kGgGateUp ? n0 + (r & (BN / 2 - 1)) : n0 + r;
    const size_t ebase = (size_t)e * args.N;
    rbq[i] = gg_rsrc(reinterpret_cast<const char*>(bm.q) + ebase * qrow, (uint32_t)args.N * qrow);
    rbs[i] = gg_rsrc(static_cast<const char*>(bm.scales) + ebase * srow, (uint32_t)args.N * srow);
    rbb[i] = gg_rsrc(static_cast<const char*>(bm.biases) + ebase * srow, (uint32_t)args.N * srow);
    const bool ok = bn < args.N;
    b_qoff[i] = ok ? (uint32_t)bn * qrow + (q % CPR_B) * 16 : kOob;
    b_soff[i] = ok ? (uint32_t)bn * srow : kOob;
  }

  // SL: the tile's weight rows fall into HALVES contiguous row ranges of the
  // scale and bias matrices (gate/up: BN/2 gate rows, then BN/2 up rows;
  // otherwise BN rows of one matrix). Each range is copied into LDS in 1 KB
  // pieces at a 1 KB-aligned offset (HS bytes apart), so the zeros or
  // neighbouring rows that a partial last piece brings in land in padding.
  // Rows past N read as zero. Per K step a thread then reads its row's scale
  // and bias from LDS instead of two 2-byte loads from 64 different rows.
  constexpr int HALVES = MODE == kGgGateUp ? 2 : 1;
  constexpr int HROWS = BN / HALVES;
  const int G = args.Kin / BK;
  const int hbytes = HROWS * G * 2;
  const int hs = (hbytes + 1023) & ~1023;
  int sidx[LB];
  if constexpr (SL) {
#pragma unroll
    for (int h = 0; h < HALVES; ++h) {
      const tfm_affine& bm = h ? args.wb : args.wa;
      const size_t ebase = (size_t)e * args.N;
      const auto rs = gg_rsrc(static_cast<const char*>(bm.scales) + ebase * srow, (uint32_t)args.N * srow);
      const auto rb = gg_rsrc(static_cast<const char*>(bm.biases) + ebase * srow, (uint32_t)args.N * srow);
      const uint32_t g0 = (uint32_t)n0 * srow;
      for (int c = wave; c * 1024 < hbytes; c += C::WAVES) {
        lds_dma16(rs, sSc + (h * hs + c * 1024) / 2, g0 + c * 1024 + lane * 16, 0);
        lds_dma16(rb, sBi + (h * hs + c * 1024) / 2, g0 + c * 1024 + lane * 16, 0);
      }
    }
#pragma unroll
    for (int i = 0; i < LB; ++i) {
      const int r = (i * T + tid) / CPR_B;
      sidx[i] = (r / HROWS) * (hs / 2) + (r % HROWS) * G;
    }
  }
  // Packed codes of step kt (and, without SL, its scale and bias).
  auto bload_q = [&](RawB<LB>& st, int kt) {
    const bool live = kt < KT;
#pragma unroll
    for (int i = 0; i < LB; ++i) {
      st.b[i] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(live ? rbq[i] : rnull, b_qoff[i], kt * (BK * BITS / 8), 0));
      if constexpr (!SL) {
        st.s[i] = __builtin_amdgcn_raw_buffer_load_b16(live ? rbs[i] : rnull, b_soff[i], kt * 2, 0);
        st.bias[i] = __builtin_amdgcn_raw_buffer_load_b16(live ? rbb[i] : rnull, b_soff[i], kt * 2, 0);
      }
    }
  };
  // SL: scale and bias of step kt from LDS (steps past the end reuse the
  // last group; their codes and activations are zero).
  auto bload_sb = [&](RawB<LB>& st, int kt) {
    if constexpr (SL) {
      const int g = kt < KT ? kt : KT - 1;
#pragma unroll
      for (int i = 0; i < LB; ++i) {
        st.s[i] = sSc[sidx[i] + g];
        st.bias[i] = sBi[sidx[i] + g];
      }
    }
  };
  auto bload = [&](RawB<LB>& st, int kt) {
    bload_q(st, kt);
    bload_sb(st, kt);
  };
  // Word w (of LB*4) of the dequantised B step: 8 elements (one LDS chunk)
  // for 4-bit, 4 elements (half a chunk) for 8-bit.
  auto bstore_word = [&](const RawB<LB>& st, uint16_t* dst, int w) {
    const int i = w / 4, k = w % 4;
    const int q = i * T + tid;
    const float sc = st2f<F16>((uint16_t)st.s[i]), bi = st2f<F16>((uint16_t)st.bias[i]);
    if constexpr (BITS == 4) {
      const uint4 pk = dequant_word<F16>(word_of(st.b[i], k), sc, bi);
      *reinterpret_cast<uint4*>(&dst[swz(q >> 1, (q & 1) * 4 + k)]) = pk;
    } else {
      const uint2 pk = dequant_word_u8<F16>(word_of(st.b[i], k), sc, bi);
      *reinterpret_cast<uint2*>(&dst[swz(q >> 2, (q & 3) * 2 + (k >> 1)) + (k & 1) * 4]) = pk;
    }
  };

  // ---- wave tile ----
  const int wm = wave / C::WAVES_N, wn = wave % C::WAVES_N;
  int brow[NB];
#pragma unroll
  for (int j = 0; j < NB; ++j) {
    if (MODE == kGgGateUp)
      brow[j] = j < NB / 2 ? wn * (C::WN / 2) + j * 32 : BN / 2 + wn * (C::WN / 2) + (j - NB / 2) * 32;
    else
      brow[j] = wn * C::WN + j * 32;
  }

  f32x16_t acc[MB][NB];
#pragma unroll
  for (int i = 0; i < MB; ++i)
#pragma unroll
    for (int j = 0; j < NB; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;

  // MFMAs of one LDS stage (fragments of K sub-step ks+1 are read during the
  // MFMAs of ks); the dequantised next B step is written during sub-steps
  // 1..3, so its loads have had more than a step to arrive.
  // MBL = the wave's 32-row blocks that hold rows of the segment (0..MB): the
  // wave reads A fragments and runs MFMAs for those blocks only. With MBL = 0
  // (every row of the wave past the segment) it skips fragment reads and
  // MFMAs altogether, which frees its SIMD's matrix pipe for the other wave
  // there, and only does its share of the loads and LDS writes.
  auto compute = [&](auto mbl_tag, const uint16_t* A, const uint16_t* Bs, const RawB<LB>& nxt,
                     uint16_t* nB) {
    constexpr int MBL = decltype(mbl_tag)::value;
    op8_t<F16> af[2][MB], bfr[2][NB];
    auto frag = [&](int ks, int slot) {
      const int kc = ks * 2 + (lane >> 5);
#pragma unroll
      for (int i = 0; i < MBL; ++i)
        af[slot][i] = *reinterpret_cast<const op8_t<F16>*>(&A[swz(wm * C::WM + i * 32 + (lane & 31), kc)]);
#pragma unroll
      for (int j = 0; j < NB; ++j)
        bfr[slot][j] = *reinterpret_cast<const op8_t<F16>*>(&Bs[swz(brow[j] + (lane & 31), kc)]);
    };
    if constexpr (MBL > 0) frag(0, 0);
    static_for<0, 4>([&](auto kc_) {
      constexpr int ks = decltype(kc_)::value;
      if constexpr (MBL > 0) {
        if constexpr (ks < 3) frag(ks + 1, (ks + 1) & 1);
#pragma unroll
        for (int i = 0; i < MBL; ++i)
#pragma unroll
          for (int j = 0; j < NB; ++j)
            acc[i][j] = mfma32<F16>(af[ks & 1][i], bfr[ks & 1][j], acc[i][j]);
      }
      if constexpr (ks >= 1) {
#pragma unroll
        for (int w = (ks - 1) * LB * 4 / 3; w < ks * LB * 4 / 3; ++w) bstore_word(nxt, nB, w);
      }
    });
  };
  // End of a step: the barrier's release fence waits for this wave's LDS
  // writes (copies and dequantised B) and its outstanding weight loads; after
  // it every wave's writes are visible.
  auto step_end = [&]() { __syncthreads(); };

  // With an odd step count the loop runs one more step on zeros (A and B
  // both read from null buffers), which adds nothing.
  RawB<LB> st0, st1;
  a_copy(sA0, 0);
  bload_q(st0, 0);
  bload_q(st1, 1);
  // SL: every wave's scale copies are complete and visible after this barrier
  if constexpr (SL) __syncthreads();
  bload_sb(st0, 0);
  bload_sb(st1, 1);
#pragma unroll
  for (int w = 0; w < LB * 4; ++w) bstore_word(st0, sB0, w);
  step_end();
  auto main_loop = [&](auto mbl_tag) {
    for (int kt = 0; kt < KT; kt += 2) {
      a_copy(sA1, kt + 1);
      bload(st0, kt + 2);
      __builtin_amdgcn_sched_barrier(0);
      compute(mbl_tag, sA0, sB0, st1, sB1);
      step_end();
      a_copy(sA0, kt + 2);
      bload(st1, kt + 3);
      __builtin_amdgcn_sched_barrier(0);
      compute(mbl_tag, sA1, sB1, st0, sB0);
      step_end();
    }
  };
  // Live row blocks of this wave (wave-uniform), one compiled loop per count.
  static_assert(MB == 2 || MB == 4, "row blocks per wave");
  const int live_rows = rows_valid - wm * C::WM;
  const int mbl = live_rows <= 0 ? 0 : min(MB, (live_rows + 31) / 32);
  if (mbl == MB) {
    main_loop(std::integral_constant<int, MB>{});
  } else if constexpr (MB == 4) {
    if (mbl == 3)
      main_loop(std::integral_constant<int, 3>{});
    else if (mbl == 2)
      main_loop(std::integral_constant<int, 2>{});
    else if (mbl == 1)
      main_loop(std::integral_constant<int, 1>{});
    else
      main_loop(std::integral_constant<int, 0>{});
  } else {
    if (mbl == 1)
      main_loop(std::integral_constant<int, 1>{});
    else
      main_loop(std::integral_constant<int, 0>{});
  }

  // ---- epilogue ----
  // Private staging block of this wave: 32 rows x SROW bf16 inside one of the
  // four stages (every wave is past the last barrier, so LDS is free).
  uint16_t* stage = (wave & 3) == 0 ? sA0 : (wave & 3) == 1 ? sA1 : (wave & 3) == 2 ? sB0 : sB1;
  stage += (wave >> 2) * 32 * C::SROW;
  constexpr int CPR = C::WCOLS / 8;             // 16-byte chunks per staged row
  const int col_base = MODE == kGgGateUp ? n0 + wn * (C::WN / 2) : n0 + wn * C::WN;
  // Row blocks by compile-time index (a runtime loop with an early exit can
  // leave acc dynamically indexed, and then in scratch memory).
  static_for<0, MB>([&](auto ic) {
    constexpr int i = decltype(ic)::value;
    const int r0 = wm * C::WM + i * 32;         // first tile row of this block
    if (r0 >= rows_valid) return;
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      const int rr = acc_row(v, lane);
      if (MODE == kGgGateUp) {
#pragma unroll
        for (int jb = 0; jb < NB / 2; ++jb)
          stage[rr * C::SROW + jb * 32 + (lane & 31)] = f2st<F16>(swiglu(acc[i][jb][v], acc[i][jb + NB / 2][v]));
      } else {
#pragma unroll
        for (int jb = 0; jb < NB; ++jb) stage[rr * C::SROW + jb * 32 + (lane & 31)] = f2st<F16>(acc[i][jb][v]);
      }
    }
    // Same-wave LDS accesses complete in order: the reads see the writes.
#pragma unroll
    for (int c0 = 0; c0 < 32 * CPR; c0 += 64) {
      const int c = c0 + lane;
      const int row = c / CPR, part = c % CPR;
      const int rr = r0 + row;
      const int n = col_base + part * 8;
      if (c < 32 * CPR && rr < rows_valid && n < args.N) {
        const uint4 v = *reinterpret_cast<const uint4*>(&stage[row * C::SROW + part * 8]);
        const int j = m0 + rr;
        const int64_t orow = MODE == kGgPlain ? (int64_t)route_flat(args.rm, j) : (int64_t)j;
        *reinterpret_cast<uint4*>(&args.out[orow * args.N + n]) = v;
      }
    }
  });
}

// Tile shapes (eight waves each): 256 x 256 (2 x 4 waves of 128 x 64) when
// the experts hold enough routes to fill 256-row tiles, 128 x 256 (2 x 4
// waves of 64 x 64) otherwise. TFM_GGEMM_TILE=256 or 128 forces one of them.
// ---------------------------------------------------------------------------
// 4-bit weights with inputs up to 2048 wide, a multiple of 128: the weights
// stay in registers.
//
// Tile: BM routed rows x 256 weight rows, eight waves. Wave w owns 32 weight
// rows (gate/up: gate rows 16w..16w+15 and the same up rows; down and plain:
// rows 32w..32w+31) for all BM rows, as 16 x 16 blocks of
// v_mfma_f32_16x16x32_bf16 (or _f16): BM/16 row blocks x 2 column blocks,
// 4 fp32 accumulators each per lane. A gate block and its up block sit in
// the same lanes, so SwiGLU needs no exchange.
//
// Per super-step of 128 k (two quantisation groups):
//   * the BM activation rows are copied into LDS (one of two stages);
//   * lane l loads 16 contiguous bytes (32 codes) of each of its two weight
//     rows: k = 32 (l / 16) .. + 31 of the super-step, which share one scale
//     group. Word s of them (k = 32 (l / 16) + 8 s .. + 7) is dequantised
//     into the B operand of sub-step s. The reduction order inside an MFMA is
//     free, so the A operand of sub-step s for lane l is the same k range:
//     LDS chunk 4 (l / 16) + s of the row;
//   * one barrier, for the next stage's activations.
// Every packed weight is dequantised exactly once per tile and never goes
// through LDS; scales and biases of the tile's rows are copied into LDS once
// per tile. Per 128 k a wave runs 4 x BM/8 MFMAs for one barrier, twice the
// work per barrier of the kernel above.
//
// LDS: activation row r of a stage is 256 B (16 chunks of 16 B); chunk c is
// stored in slot c ^ (r & 15), so the 16 lanes of one read pass (16
// consecutive rows, one chunk) hit distinct bank groups.
constexpr int BK2 = 128;

__device__ __forceinline__ f32x4_t mfma16(bf16x8_t a, bf16x8_t b, f32x4_t c, std::false_type) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x4_t mfma16(f16x8_t a, f16x8_t b, f32x4_t c, std::true_type) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// BM = 64 (few routes per expert): 64 KB of LDS and 32 accumulator
// registers, so two workgroups share a compute unit and each covers the
// other's weight-load latency, which a super-step's few MFMAs cannot. WV = 4
// (64-row tiles only) halves the weight rows of a tile (128: 64 gate and 64
// up rows, or 128 down rows) for twice the tiles, where 8-wave tiles would
// leave compute units idle (a few experts or a few output columns: Granite
// decode batches, a dense matrix); 48 KB of LDS, three workgroups per
// compute unit.
template <int BM, int MODE, bool F16, int WV, bool FEW = false>
__global__ __launch_bounds__(WV * 64, BM == 64 ? (WV == 8 ? 2 : 3) : 1) void ggemm_wr_kernel(GgArgs args) {
  constexpr int WAVES = WV, BN = 32 * WV;
  constexpr int MB = BM / 16;                     // 16-row blocks per wave
  constexpr int OUT_COLS = MODE == kGgGateUp ? BN / 2 : BN;
  constexpr int LA = BM / (4 * WAVES);            // 4-row (1 KB) copies per wave per super-step
  static_assert(WV == 8 || (WV == 4 && BM == 64), "8 waves, or 4 with 64-row tiles");
  static_assert(LA >= 1, "every wave copies activation rows");
  constexpr int SROW = 136;                       // epilogue staging row stride (128 columns + 16 B)
  constexpr int HALF_ROWS = BM / 2;               // staged rows per activation stage
  static_assert(BM == 64 || BM == 128 || BM == 256, "tile rows");
  static_assert(HALF_ROWS * SROW <= BM * BK2, "epilogue staging fits a stage");
  using op_t = op8_t<F16>;
  using f16tag = std::integral_constant<bool, F16>;

  __shared__ __attribute__((aligned(16))) uint16_t sA0[BM * BK2];
  __shared__ __attribute__((aligned(16))) uint16_t sA1[BM * BK2];
  __shared__ __attribute__((aligned(16))) uint16_t sSc[BN * 32];
  __shared__ __attribute__((aligned(16))) uint16_t sBi[BN * 32];
  // Tile prefix, XCD bounds and expert index: in activation stage 1, first
  // written after the prologue's barrier.
  int* const s_tiles = reinterpret_cast<int*>(sA1);
  int* const s_bound = s_tiles + 66;
  int& s_expert = s_tiles[65];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int E = args.g.E;
  const int NT = (args.N + OUT_COLS - 1) / OUT_COLS;
  const int xcd = blockIdx.x & 7;
  const int local = blockIdx.x >> 3;

  // Tiles in m-major order (experts in order, their m-tiles, n-tiles
  // innermost). Workgroups are dispatched round-robin over the 8 XCDs; XCD
  // x takes a contiguous run of the order (its n-tiles and neighbouring
  // m-tiles share activations and weights in its L2) holding about 1/8 of
  // the estimated work. With 256-row tiles a tile costs about 13 + (live
  // 16-row blocks) units (measured: 23.6 + 1.85 x blocks microseconds at
  // 4096 tokens), so runs of short tiles are longer; 128-row tiles cost
  // about the same whatever their rows, and count one unit each.
  constexpr bool BAL = BM == 256;
  constexpr int CF = BAL ? 13 + MB : 1;
  if (tid < 64) {
    int cnt = 0;
    if (tid < E) cnt = grp_offset(args.g, tid + 1) - grp_offset(args.g, tid);
    const int full = cnt / BM, part = cnt % BM;
    const int cp = part > 0 ? (BAL ? 13 + min(MB, ((part + 63) / 64) * 4) : 1) : 0;
    const int mt_e = full + (part > 0 ? 1 : 0);
    const int cost_e = NT * (full * CF + cp);
    int mt_i = mt_e, cost_i = cost_e;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      const int o1 = __shfl_up(mt_i, d, 64), o2 = __shfl_up(cost_i, d, 64);
      if (lane >= d) {
        mt_i += o1;
        cost_i += o2;
      }
    }
    s_tiles[tid + 1] = mt_i;
    if (tid == 0) s_tiles[0] = 0;
    const int W = __shfl(cost_i, 63, 64);
    // bound k: tiles whose start lies below target (xcd + k) W / 8
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      const int T = (int)(((int64_t)(xcd + k) * W) / 8);
      if (tid == 0) s_bound[k] = 0;
      const int pc = cost_i - cost_e;
      if (tid < E && pc < T && T <= cost_i) {
        const int rel = T - pc, fc = full * NT * CF;
        const int c = rel <= fc ? (rel + CF - 1) / CF : full * NT + (rel - fc + cp - 1) / cp;
        s_bound[k] = (mt_i - mt_e) * NT + c;
      }
    }
  }
  __syncthreads();
  const int ti = s_bound[0] + local;
  if (ti >= s_bound[1]) return;
  const int mt = ti / NT, nt = ti % NT;
  if (tid < E && s_tiles[tid] <= mt && mt < s_tiles[tid + 1]) s_expert = tid;
  __syncthreads();
  const int e = s_expert;
  const int seg0 = grp_offset(args.g, e), seg1 = grp_offset(args.g, e + 1);
  const int m0 = seg0 + (mt - s_tiles[e]) * BM;
  const int rows_valid = min(BM, seg1 - m0);
  const int n0 = nt * OUT_COLS;
  const int KT = args.Kin / BK2;
  const int G = args.Kin / BK;                    // quantisation groups per row

  // ---- activations: global -> LDS ----
  // Copy i of wave w: rows 4 (WAVES i + w) .. + 3 (copy i of all waves
  // together: rows 4 WAVES i .. + 4 WAVES - 1); lane l writes slot l % 16 of
  // row 4 (WAVES i + w) + l / 16, which holds chunk (l % 16) ^ (row & 15).
  const __amdgpu_buffer_rsrc_t ra = gg_rsrc(args.x, args.x_bytes);
  const __amdgpu_buffer_rsrc_t rnull = gg_rsrc(args.x, 0);
  uint32_t a_off[LA];
#pragma unroll
  for (int i = 0; i < LA; ++i) {
    const int r = 4 * (WAVES * i + wave) + (lane >> 4);
    const int c = (lane & 15) ^ (r & 15);
    if (r < rows_valid) {
      const int64_t src = MODE == kGgDown ? (int64_t)(m0 + r) : route_row(args.rm, m0 + r);
      a_off[i] = (uint32_t)((src * args.Kin + c * 8) * 2);
    } else {
      a_off[i] = kOob;
    }
  }
  auto a_copy = [&](uint16_t* dst, int kt) {
    const __amdgpu_buffer_rsrc_t r = kt < KT ? ra : rnull;
#pragma unroll
    for (int i = 0; i < LA; ++i) lds_dma16(r, dst + 4 * (WAVES * i + wave) * BK2, a_off[i], kt * BK2 * 2);
  };
  // Copy i alone (the main loop spreads the copies over a super-step).
  auto a_copy1 = [&](uint16_t* dst, int kt, auto i_) {
    constexpr int i = decltype(i_)::value;
    const __amdgpu_buffer_rsrc_t r = kt < KT ? ra : rnull;
    lds_dma16(r, dst + 4 * (WAVES * i + wave) * BK2, a_off[i], kt * BK2 * 2);
  };

  // ---- weights ----
  const int g4 = lane >> 4;                       // k quarter of the super-step
  const uint32_t qrow = (uint32_t)args.Kin / 2, srow = (uint32_t)G * 2;
  __amdgpu_buffer_rsrc_t rbq[2];
  uint32_t b_qoff[2];
  int trow[2];                                    // weight row within the tile (0..255)
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const tfm_affine& bm = (MODE == kGgGateUp && j == 1) ? args.wb : args.wa;
    trow[j] = MODE == kGgGateUp ? j * (BN / 2) + 16 * wave + (lane & 15) : 32 * wave + 16 * j + (lane & 15);
    const int bn = MODE == kGgGateUp ? n0 + 16 * wave + (lane & 15) : n0 + 32 * wave + 16 * j + (lane & 15);
    rbq[j] = gg_rsrc(reinterpret_cast<const char*>(bm.q) + (size_t)e * args.N * qrow, (uint32_t)args.N * qrow);
    b_qoff[j] = bn < args.N ? (uint32_t)bn * qrow + 16u * g4 : kOob;
  }
  auto bload = [&](uint4* raw, int kt) {
    const bool live = kt < KT;
#pragma unroll
    for (int j = 0; j < 2; ++j)
      raw[j] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(live ? rbq[j] : rnull, b_qoff[j], kt * 64, 0));
  };

  // Scales and biases of the tile's rows, copied once: HALVES contiguous row
  // ranges, each at a 1 KB-aligned offset, row r of a range at r * 2G bytes.
  // sb_read reads one group of 16 consecutive rows per instruction; at a row
  // stride of 2G bytes those rows share 2 to 4 banks (32 or 64 banks of 4
  // bytes). The layouts move row r's group-pair dword d to d ^ sw(r):
  //  * kSbPlain: sw = 0, copied as contiguous 16-byte pieces;
  //  * kSbDword: sw(r) = (r G / 64) mod (G/2) for G/2 a power of two, which
  //    puts the 16 rows in 16 banks; copied with 4-byte LDS-DMA, the swizzle
  //    applied to the source offsets;
  //  * kSbChunk (G = 16 or 32): 16-byte pieces of a row swapped,
  //    sw(r) = 4 ((r / 4) mod (G/8)): 2 rows per bank at worst, and the copy
  //    stays 16-byte LDS-DMA.
  constexpr int HALVES = MODE == kGgGateUp ? 2 : 1;
  constexpr int HROWS = BN / HALVES;
  const int GH = G / 2;                           // group-pair dwords per row
  const int CH = G / 8;                           // 16-byte pieces per row
  const int lay = args.sb_layout;
  const int swm = (GH & (GH - 1)) == 0 ? GH - 1 : 0;
  auto sb_swz = [&](int r) {
    return lay == kSbDword ? ((r * G) >> 6) & swm : lay == kSbChunk ? ((r >> 2) & (CH - 1)) << 2 : 0;
  };
  const int hbytes = HROWS * G * 2;
  const int hs = (hbytes + 1023) & ~1023;
#pragma unroll
  for (int h = 0; h < HALVES; ++h) {
    const tfm_affine& bm = h ? args.wb : args.wa;
    const size_t ebase = (size_t)e * args.N;
    const auto rs = gg_rsrc(static_cast<const char*>(bm.scales) + ebase * srow, (uint32_t)args.N * srow);
    const auto rb = gg_rsrc(static_cast<const char*>(bm.biases) + ebase * srow, (uint32_t)args.N * srow);
    const uint32_t g0 = (uint32_t)n0 * srow;
    if (lay == kSbDword) {
      for (int c = wave; c * 256 < hbytes; c += WAVES) {
        const int p = 64 * c + lane;              // destination dword of the range
        const int r = p / GH, x = p - r * GH;
        const uint32_t src = 4 * p < hbytes ? g0 + (uint32_t)r * srow + 4u * (uint32_t)(x ^ sb_swz(r)) : kOob;
        lds_dma4(rs, sSc + (h * hs + c * 256) / 2, src);
        lds_dma4(rb, sBi + (h * hs + c * 256) / 2, src);
      }
    } else {
      for (int c = wave; c * 1024 < hbytes; c += WAVES) {
        uint32_t src = g0 + c * 1024 + lane * 16;
        if (lay == kSbChunk) {
          const int p = 64 * c + lane;            // destination 16-byte piece of the range
          const int r = p / CH, x = p - r * CH;
          src = 16 * p < hbytes ? g0 + (uint32_t)r * srow + 16u * (uint32_t)(x ^ (sb_swz(r) >> 2)) : kOob;
        }
        lds_dma16(rs, sSc + (h * hs + c * 1024) / 2, src, 0);
        lds_dma16(rb, sBi + (h * hs + c * 1024) / 2, src, 0);
      }
    }
  }
  int sidx[2], ssw[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    sidx[j] = (trow[j] / HROWS) * (hs / 2) + (trow[j] % HROWS) * G;
    ssw[j] = sb_swz(trow[j] % HROWS);
  }
  // scale and bias of super-step kt for both rows (past the end: last group)
  auto sb_read = [&](float* sc, float* bi, int kt) {
    int g = 2 * kt + (g4 >> 1);
    g = g < G ? g : G - 1;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int o = sidx[j] + 2 * ((g >> 1) ^ ssw[j]) + (g & 1);
      sc[j] = st2f<F16>(sSc[o]);
      bi[j] = st2f<F16>(sBi[o]);
    }
  };
  auto deq = [&](op_t* b, const uint4* raw, const float* sc, const float* bi, int s) {
#pragma unroll
    for (int j = 0; j < 2; ++j) b[j] = __builtin_bit_cast(op_t, dequant_word<F16>(word_of(raw[j], s), sc[j], bi[j]));
  };

  f32x4_t acc[MB][2];
#pragma unroll
  for (int i = 0; i < MB; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};

  // One super-step on activation stage A: sub-step s runs the MFMAs of the
  // MBL live row blocks with B operand b (word s) and dequantises the B
  // operand of the next sub-step (word s + 1, or word 0 of the next
  // super-step's raw weights). The (sub-step, row block) pairs run as one
  // compile-time sequence with the A fragment of pair q + D read while pair
  // q computes (a ring of D + 1 fragments); the scheduler is asked for the
  // first D reads, then per pair two MFMAs, the read D pairs ahead and three
  // VALU instructions. The activation copies of the next super-step (into
  // stage An) are issued one every STEP pairs over the first half of the
  // sequence: issued together they would hold the wave at the address unit,
  // with no MFMAs issued, for most of a thousand cycles. Only the NC copies
  // of rows below 16 MBL are issued: the other rows are never read.
  // Fragment address of row block i, sub-step s: the lane's byte offset
  // (row lane % 16, slot (4 g4) ^ (lane % 16)) XOR 16 s, plus 4096 i. The
  // lane offset is made opaque per super-step so that the four per-sub-step
  // addresses are formed there instead of being held across the loop.
  const uint32_t a_lane = (uint32_t)((lane & 15) * BK2 * 2 + (((4 * g4) ^ (lane & 15)) << 4));
  auto compute = [&](auto mbl_tag, const uint16_t* A, op_t* b, const uint4* rc, const float* sc,
                     const float* bic, const uint4* rn, const float* sn, const float* bin, uint16_t* An,
                     int ktn, auto after_copy) __attribute__((always_inline)) {
    constexpr int MBL = decltype(mbl_tag)::value;
    constexpr int NQ = 4 * MBL, D = 3, R = D + 1;
    constexpr int CR = 4 * WAVES;  // rows per copy round
    constexpr int NC = (16 * MBL + CR - 1) / CR < LA ? (16 * MBL + CR - 1) / CR : LA;
    constexpr int STEP = NQ / (2 * NC) > 0 ? NQ / (2 * NC) : 1;
    static_assert(STEP * (NC - 1) < NQ, "every copy is issued");
    op_t af[R];
    uint32_t nbw[2][4];                           // next B operand, packed pairs
    uint32_t lo[2], hi[2];                        // nibble bytes of the word being dequantised
    float f[16];
    uint32_t al = a_lane;
    asm volatile("" : "+v"(al));
    const char* const Ab = reinterpret_cast<const char*>(A);
    auto rd = [&](auto q_) {
      constexpr int q = decltype(q_)::value, s = q / MBL, i = q % MBL;
      af[q % R] = *reinterpret_cast<const op_t*>(Ab + (al ^ (16u * s)) + 16 * BK2 * 2 * i);
    };
    static_for<0, D>([&](auto q_) { rd(q_); });
    __builtin_amdgcn_sched_barrier(0);
    static_for<0, NQ>([&](auto q_) {
      constexpr int q = decltype(q_)::value, s = q / MBL, i = q % MBL;
      if constexpr (q % STEP == 0 && q / STEP < NC) a_copy1(An, ktn, std::integral_constant<int, q / STEP>{});
      if constexpr (q == STEP * (NC - 1)) after_copy();
      if constexpr (q + D < NQ) rd(std::integral_constant<int, q + D>{});
      acc[i][0] = mfma16(af[q % R], b[0], acc[i][0], f16tag{});
      acc[i][1] = mfma16(af[q % R], b[1], acc[i][1], f16tag{});
      // Slice of the next sub-step's B operand: codes c0..c1-1 of the 16
      // (code c: row j = c / 8, element c % 8 of word s + 1, or word 0 of
      // the next super-step's raw weights).
      constexpr int c0 = 16 * i / MBL, c1 = 16 * (i + 1) / MBL;
      static_for<c0, c1>([&](auto c_) {
        constexpr int c = decltype(c_)::value, j = c / 8, el = c % 8;
        const uint32_t* rw = s < 3 ? reinterpret_cast<const uint32_t*>(&rc[j]) : reinterpret_cast<const uint32_t*>(&rn[j]);
        const float scj = s < 3 ? sc[j] : sn[j], bij = s < 3 ? bic[j] : bin[j];
        if constexpr (el == 0) {
          const uint32_t w = rw[s < 3 ? s + 1 : 0];
          lo[j] = w & 0x0f0f0f0fu;
          hi[j] = (w >> 4) & 0x0f0f0f0fu;
          asm("" : "+v"(lo[j]));
          asm("" : "+v"(hi[j]));
        }
        const uint32_t src = (el & 1) ? hi[j] : lo[j];
        f[c] = __builtin_fmaf(scj, (float)((src >> (8 * (el >> 1))) & 0xffu), bij);
        if constexpr (el & 1) nbw[j][el >> 1] = pack_st2<F16>(f[c - 1], f[c]);
      });
      if constexpr (i == MBL - 1) {
#pragma unroll
        for (int j = 0; j < 2; ++j)
          b[j] = __builtin_bit_cast(op_t, make_uint4(nbw[j][0], nbw[j][1], nbw[j][2], nbw[j][3]));
      }
      __builtin_amdgcn_sched_barrier(0);
    });
  };

  // ---- few rows (FEW instances): weights two super-steps ahead ----
  // In the loop below every super-step ends at a barrier that waits for all
  // of its loads, and the raw weights of super-step k+1 (whose first word
  // the last sub-step of super-step k dequantises) are requested at the start
  // of super-step k: one super-step of loads in flight. A tile of at most 16
  // rows (one row block) has too few MFMAs per super-step to cover a memory
  // latency that way. Here the raw weights of super-step k+2 are requested
  // right after the activation copy of super-step k+1, and the barrier waits
  // only for that copy (the vector memory counter retires in issue order), so
  // they stay in flight across it. The products and their order are those of
  // the loop below.
  if (FEW && rows_valid <= 16 && (KT & 3) == 0) {
    if constexpr (FEW) {
      static_assert(BM == 64, "few-row tiles are 64-row tiles");
      uint4 rw[4][2];                             // raw weights of super-step k in slot k % 4
      float fsc[2][2], fbi[2][2];                 // scales and biases of super-step k in set k % 2
      op_t fb[2];
      a_copy(sA0, 0);
      bload(rw[0], 0);
      bload(rw[1], 1);
      __syncthreads();  // scale copies and stage 0 complete and visible
      sb_read(fsc[0], fbi[0], 0);
      deq(fb, rw[0], fsc[0], fbi[0], 0);
      for (int kt0 = 0; kt0 < KT; kt0 += 4) {
        static_for<0, 4>([&](auto q_) {
          constexpr int q = decltype(q_)::value, c = q % 2, n = 1 - c;
          const int kt = kt0 + q;
          uint16_t* const A = c == 0 ? sA0 : sA1;
          uint16_t* const An = c == 0 ? sA1 : sA0;
          sb_read(fsc[n], fbi[n], kt + 1);
          __builtin_amdgcn_sched_barrier(0);
          compute(std::integral_constant<int, 1>{}, A, fb, rw[q], fsc[c], fbi[c], rw[(q + 1) % 4], fsc[n],
                  fbi[n], An, kt + 1, [&] { bload(rw[(q + 2) % 4], kt + 2); });
          // This wave's copy into An is done (only the two weight loads
          // issued after it may be outstanding), then every wave's.
          asm volatile("s_waitcnt vmcnt(2)\n\ts_barrier" ::: "memory");
        });
      }
    }
  } else {
  // ---- prologue ----
  uint4 r0[2], r1[2];
  float sc0[2], bi0[2], sc1[2], bi1[2];
  op_t bop[2];
  a_copy(sA0, 0);
  bload(r0, 0);
  __syncthreads();  // scale copies and stage 0 complete and visible
  sb_read(sc0, bi0, 0);
  deq(bop, r0, sc0, bi0, 0);

  // Super-step S: load the raw weights of S+1 and read its scales, compute
  // (copying S+1 into the other stage on the way), barrier. With an odd
  // count the loop runs one more super-step on zero activations.
  auto main_loop = [&](auto mbl_tag) {
    for (int kt = 0; kt < KT; kt += 2) {
      bload(r1, kt + 1);
      sb_read(sc1, bi1, kt + 1);
      __builtin_amdgcn_sched_barrier(0);
      compute(mbl_tag, sA0, bop, r0, sc0, bi0, r1, sc1, bi1, sA1, kt + 1, [] {});
      __syncthreads();
      bload(r0, kt + 2);
      sb_read(sc0, bi0, kt + 2);
      __builtin_amdgcn_sched_barrier(0);
      compute(mbl_tag, sA1, bop, r1, sc1, bi1, r0, sc0, bi0, sA0, kt + 2, [] {});
      __syncthreads();
    }
  };
  // Live row blocks (uniform over the workgroup), in steps of four (with
  // 64-row tiles: 1, 2 or 4).
  const int live = min(MB, ((rows_valid + 63) / 64) * 4);
  if constexpr (MB == 16) {
    if (live == 16)
      main_loop(std::integral_constant<int, 16>{});
    else if (live == 12)
      main_loop(std::integral_constant<int, 12>{});
    else if (live == 8)
      main_loop(std::integral_constant<int, 8>{});
    else
      main_loop(std::integral_constant<int, 4>{});
  } else if constexpr (MB == 8) {
    if (live == 8)
      main_loop(std::integral_constant<int, 8>{});
    else
      main_loop(std::integral_constant<int, 4>{});
  } else {
    // 64-row tiles (few routes per expert): one or two live blocks when the
    // tile holds at most 16 or 32 rows, so that empty rows cost no MFMAs.
    if (rows_valid <= 16)
      main_loop(std::integral_constant<int, 1>{});
    else if (rows_valid <= 32)
      main_loop(std::integral_constant<int, 2>{});
    else
      main_loop(std::integral_constant<int, 4>{});
  }
  }

  // ---- epilogue ----
  // Rows staged row-major, CP columns per pass (the first BM/2 rows in
  // stage 0, the rest in stage 1), then written as 16-byte row pieces.
  // Gate/up: one pass of BN/2 columns (wave w holds columns 16w..16w+15
  // after SwiGLU); down and plain: BN/128 passes of 128 columns, waves
  // 4p..4p+3 staging columns 128p..128p+127.
  constexpr int PASSES = MODE == kGgGateUp ? 1 : BN / 128;
  constexpr int CP = MODE == kGgGateUp ? BN / 2 : 128;
  constexpr int PARTS = CP / 8;                   // 16-byte pieces per staged row
  constexpr int RPI = WAVES * 64 / PARTS;         // rows written per iteration
  static_assert(CP + 8 <= SROW, "staged row fits its stride");
  static_for<0, PASSES>([&](auto p_) {
    constexpr int p = decltype(p_)::value;
    if (p > 0) __syncthreads();  // the previous pass's reads are done
    const bool mine = MODE == kGgGateUp || (wave >> 2) == p;
    if (mine) {
      static_for<0, MB>([&](auto i_) {
        constexpr int i = decltype(i_)::value;
        if (16 * i >= rows_valid) return;
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const int row = 16 * i + 4 * g4 + v;
          uint16_t* st = (row < HALF_ROWS ? sA0 : sA1) + (row % HALF_ROWS) * SROW;
          if constexpr (MODE == kGgGateUp) {
            st[16 * wave + (lane & 15)] = f2st<F16>(swiglu(acc[i][0][v], acc[i][1][v]));
          } else {
#pragma unroll
            for (int j = 0; j < 2; ++j) st[32 * (wave & 3) + 16 * j + (lane & 15)] = f2st<F16>(acc[i][j][v]);
          }
        }
      });
    }
    __syncthreads();
    const int part = tid % PARTS;
    const int n = n0 + CP * p + part * 8;
#pragma unroll
    for (int r0i = 0; r0i < BM; r0i += RPI) {
      const int row = r0i + tid / PARTS;
      if (row < rows_valid && n < args.N) {
        const uint16_t* st = (row < HALF_ROWS ? sA0 : sA1) + (row % HALF_ROWS) * SROW;
        const uint4 v = *reinterpret_cast<const uint4*>(&st[part * 8]);
        const int j = m0 + row;
        const int64_t orow = MODE == kGgPlain ? (int64_t)route_flat(args.rm, j) : (int64_t)j;
        *reinterpret_cast<uint4*>(&args.out[orow * args.N + n]) = v;
      }
    }
  });
}

static int tile_override() {
  static int v = [] {
    const char* s = std::getenv("TFM_GGEMM_TILE");
    return s ? std::atoi(s) : 0;
  }();
  return v;
}

// Tile rows of the down GEMM alone (TFM_GGEMM_DOWN_TILE=64/128/256, for
// measurement; TFM_GGEMM_TILE takes precedence); 0 when unset.
static int down_tile_override() {
  static int v = [] {
    const char* s = std::getenv("TFM_GGEMM_DOWN_TILE");
    const int n = s ? std::atoi(s) : 0;
    return n == 64 || n == 128 || n == 256 ? n : 0;
  }();
  return v;
}

static bool use_tall(int64_t n_routes, int E) {
  const int o = tile_override();
  if (o == 256) return true;
  if (o == 128 || o == 64) return false;
  return n_routes >= (int64_t)E * 384;
}

static int gg_device_cus() {
  static int cus = [] {
    int dev = 0, n = 0;
    if (hipGetDevice(&dev) != hipSuccess) return 256;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
      return 256;
    return n;
  }();
  return cus;
}

// Tile rows of the weights-in-registers kernel (TFM_GGEMM_TILE=64/128/256
// forces one), from the average routes per expert a = n_routes / E and the
// tile count, with every expert's routes taken as a:
//  * 64 while a <= 56: every m-tile streams its expert's weights again, so
//    64-row tiles pay only while few experts pass 64 routes (OLMoE 33-384
//    tokens 12% faster than 128-row tiles, level at 512, 9% slower at 768;
//    Granite 256 tokens, a = 51: 58.6 against 62.6 us per layer);
//  * 256 from a = 208: a 256-row tile dequantises its weights once for twice
//    the rows (OLMoE 1792 tokens, a = 224: 309 against 319 us; 2048 tokens:
//    305 against 331; at a = 192, 1536 tokens, 128-row tiles win, 265
//    against 277);
//  * 256 below that when 256-row tiles fit one round of the compute units and
//    128-row tiles do not (Granite, 4 gate/up column tiles: 768 tokens,
//    a = 154, 84.4 against 98.6 us; at 512 tokens both fit, and 128-row tiles
//    win, 70.7 against 73.1);
//  * else 128;
//  * with few experts and output columns (E x col_tiles below a quarter of
//    the compute units: a dense matrix, E = 1), the largest tile whose count
//    fills the compute units, else 64 (OLMoE q_proj at 512 rows has 16
//    256-row tiles and 64 64-row ones).
// col_tiles: 256-row weight tiles across the output (gate/up: gate and up
// rows together).
static int wr_tile_rows(int64_t n_routes, int E, int64_t col_tiles, bool down) {
  const int o = tile_override();
  if (o == 64 || o == 128 || o == 256) return o;
  if (4 * E * col_tiles < gg_device_cus()) {
    const int64_t cus = gg_device_cus();
    for (int bm = 256; bm >= 128; bm /= 2)
      if ((n_routes + (int64_t)E * bm - 1) / ((int64_t)E * bm) * E * col_tiles >= cus) return bm;
    return 64;
  }
  if (n_routes <= (int64_t)E * 56) return 64;
  // The down GEMM keeps 64-row tiles up to 128 routes per expert: two
  // workgroups per compute unit overlap one's epilogue with the other's main
  // loop. Down GEMM, 64- against 128-row tiles: OLMoE 512 tokens 40.7 against
  // 42.8 us, 768 tokens 49.6 against 49.8, 1024 tokens 61.1 against 66.7;
  // Granite 384 tokens 17.4 against 16.4, 512 tokens 18.1 against 18.1,
  // 640 tokens 23.8 against 29.0; at OLMoE 2048 tokens (256 routes per
  // expert) 105.0 against 100.9 on 256-row tiles.
  if (down && n_routes <= (int64_t)E * 128) return 64;
  if (n_routes >= (int64_t)E * 208) return 256;
  const int64_t m128 = (n_routes + (int64_t)E * 128 - 1) / ((int64_t)E * 128);
  const int64_t m256 = (n_routes + (int64_t)E * 256 - 1) / ((int64_t)E * 256);
  const int64_t cus = gg_device_cus();
  if (E * m128 * col_tiles > cus && E * m256 * col_tiles <= cus) return 256;
  return 128;
}

static unsigned grid_for(int64_t n_routes, int E, int BM, int NT) {
  const int64_t mt_max = (n_routes + BM - 1) / BM + (n_routes < E ? n_routes : E);
  int64_t total = mt_max * NT;
  // round up to a multiple of 8 so every XCD share is complete
  total = (total + 7) / 8 * 8;
  if (total < 8) total = 8;
  return (unsigned)total;
}

template <int BM_, int BN_, int WAVES_M, int WAVES_N, int MODE, int BITS, bool F16>
static void launch_one(const GgArgs& a, int64_t n_routes, int E, hipStream_t s) {
  using C = GgCfg<BM_, BN_, WAVES_M, WAVES_N, MODE, BITS>;
  const int NT = (a.N + C::OUT_COLS - 1) / C::OUT_COLS;
  if (a.Kin <= kLdsScaleKin)
    tfm_launch(ggemm_kernel<BM_, BN_, WAVES_M, WAVES_N, MODE, BITS, F16, true>, grid_for(n_routes, E, BM_, NT), C::THREADS, 0, s, a);
  else
    tfm_launch(ggemm_kernel<BM_, BN_, WAVES_M, WAVES_N, MODE, BITS, F16, false>, grid_for(n_routes, E, BM_, NT), C::THREADS, 0, s, a);
}

// Waves per workgroup of the 64-row weights-in-registers tiles
// (TFM_GGEMM_WAVES=4/8 forces one): 4 (tiles of half the weight rows) while
// 8-wave tiles number fewer than two per compute unit, else 8. Per layer, 4
// against 8 waves: Granite decode 32 38.9 against 40.7 us, Granite 64 tokens
// 40.8 against 42.5; OLMoE 32 tokens (over two tiles per compute unit) 85.7
// against 75.2. Two-wave tiles measured no faster than four (Granite decode
// 32: 40.2 us).
static int wr_waves(int64_t tiles8) {
  static const int o = [] {
    const char* s = std::getenv("TFM_GGEMM_WAVES");
    return s ? std::atoi(s) : 0;
  }();
  if (o == 4 || o == 8) return o;
  return tiles8 < 2 * (int64_t)gg_device_cus() ? 4 : 8;
}

// Scale/bias layout of ggemm_wr_kernel for an input width (TFM_GGEMM_SB_LAYOUT
// = 0/1/2 forces kSbPlain/kSbDword/kSbChunk where it applies): kSbChunk at
// 16 and 32 groups per row, else kSbPlain. Per layer, plain / dword / chunk
// layouts on one box: OLMoE 4096 tokens (Zipf) 517.7 / 512.5 / 509.8 us
// (gate/up 274.2 / 268.9 / 267.0), 512 tokens 138.1 / 135.5 / 134.9; Granite
// 2048 tokens 156.5 / 157.4 / 156.3, decode 32 39.7 / 40.3 / 39.7.
static int sb_layout(int Kin) {
  static const int o = [] {
    const char* s = std::getenv("TFM_GGEMM_SB_LAYOUT");
    return s ? std::atoi(s) : -1;
  }();
  const int G = Kin / BK;
  if (o == kSbPlain || o == kSbDword) return o;
  return G == 16 || G == 32 ? kSbChunk : kSbPlain;
}

// The FEW instance of a 64-row launch (tiles of at most 16 rows keep their
// weights two super-steps ahead) runs where experts average at most
// kFewRowsAvg routes, so that most tiles hold at most 16 rows.
// TFM_GGEMM_FEW_ROWS=0 never uses it, =2 uses it for every 64-row launch.
constexpr int kFewRowsAvg = 12;
static bool use_few_rows(int64_t n_routes, int E) {
  static const int v = [] {
    const char* s = std::getenv("TFM_GGEMM_FEW_ROWS");
    return s && (s[0] == '0' || s[0] == '2') && s[1] == 0 ? s[0] - '0' : 1;
  }();
  return v == 2 || (v == 1 && n_routes <= (int64_t)E * kFewRowsAvg);
}

template <int BM, int MODE, bool F16, int WV>
static void launch_wr_waves(const GgArgs& a_in, int64_t n_routes, int E, hipStream_t s) {
  GgArgs a = a_in;
  a.sb_layout = sb_layout(a.Kin);
  constexpr int OUT_COLS = MODE == kGgGateUp ? 16 * WV : 32 * WV;
  const int NT = (a.N + OUT_COLS - 1) / OUT_COLS;
  // With 256-row tiles an XCD's run of cheap tiles holds more tiles than an
  // even share: at most share x 29 / 17 + 2 (full tile 29 units, cheapest
  // 17); workgroups past their XCD's run exit at once.
  unsigned grid = grid_for(n_routes, E, BM, NT);
  if (BM == 256) grid = ((grid / 8 * 29 + 16) / 17 + 2) * 8;
  // Not for 8-wave half storage: there the ring would cost a workgroup per
  // compute unit (three waves per SIMD).
  if constexpr (BM == 64 && !(F16 && WV == 8)) {
    if (use_few_rows(n_routes, E)) {
      tfm_launch(ggemm_wr_kernel<BM, MODE, F16, WV, true>, grid, WV * 64, 0, s, a);
      return;
    }
  }
  tfm_launch(ggemm_wr_kernel<BM, MODE, F16, WV>, grid, WV * 64, 0, s, a);
}

// 4-bit weights, inputs up to 2048 wide and a multiple of 128: weights in
// registers (ggemm_wr_kernel); otherwise ggemm_kernel.
template <int BM, int MODE, bool F16>
static void launch_wr(const GgArgs& a, int64_t n_routes, int E, hipStream_t s) {
  if constexpr (BM == 64) {
    constexpr int OUT8 = MODE == kGgGateUp ? 128 : 256;
    const int wv = wr_waves(grid_for(n_routes, E, BM, (a.N + OUT8 - 1) / OUT8));
    if (wv == 4) {
      launch_wr_waves<BM, MODE, F16, 4>(a, n_routes, E, s);
      return;
    }
  }
  launch_wr_waves<BM, MODE, F16, 8>(a, n_routes, E, s);
}

template <int MODE, int BITS, bool F16>
static void launch_tile(const GgArgs& a, int64_t n_routes, int E, hipStream_t s) {
#ifndef GG_NO_WR
  if constexpr (BITS == 4) {
    if (a.Kin <= kLdsScaleKin && a.Kin % BK2 == 0) {
      int bm = wr_tile_rows(n_routes, E, MODE == kGgGateUp ? (2 * (int64_t)a.N + 255) / 256 : ((int64_t)a.N + 255) / 256,
                            MODE == kGgDown);
      if (MODE == kGgDown && down_tile_override() && !tile_override()) bm = down_tile_override();
      switch (bm) {
        case 256: launch_wr<256, MODE, F16>(a, n_routes, E, s); break;
        case 64: launch_wr<64, MODE, F16>(a, n_routes, E, s); break;
        default: launch_wr<128, MODE, F16>(a, n_routes, E, s); break;
      }
      return;
    }
  }
#endif
  if (use_tall(n_routes, E))
    launch_one<256, 256, 2, 4, MODE, BITS, F16>(a, n_routes, E, s);
  else
    launch_one<128, 256, 2, 4, MODE, BITS, F16>(a, n_routes, E, s);
}

template <int MODE>
static void launch_mode(const GgArgs& a, int bits, bool f16, int64_t n_routes, int E, hipStream_t s) {
  if (bits == 8 && f16)
    launch_tile<MODE, 8, true>(a, n_routes, E, s);
  else if (bits == 8)
    launch_tile<MODE, 8, false>(a, n_routes, E, s);
  else if (f16)
    launch_tile<MODE, 4, true>(a, n_routes, E, s);
  else
    launch_tile<MODE, 4, false>(a, n_routes, E, s);
}

static void check_shapes(int N, int Kin, int bits, int64_t x_rows) {
  if (bits != 4 && bits != 8) fail(TFM_E_UNSUPPORTED, "grouped GEMM: weights must be 4-bit or 8-bit");
  if (Kin % BK != 0) fail(TFM_E_UNSUPPORTED, "grouped GEMM: input width must be a multiple of 64");
  if (N % 64 != 0) fail(TFM_E_UNSUPPORTED, "grouped GEMM: output width must be a multiple of 64");
  // Buffer offsets are 32-bit: activations and one expert's packed weights
  // must stay below 2 GiB.
  if ((double)x_rows * Kin * 2 >= 2147483648.0 || (double)N * Kin * bits / 8 >= 2147483648.0)
    fail(TFM_E_UNSUPPORTED, "grouped GEMM: operand of 2 GiB or more");
}

void launch_ggemm_gateup(const uint16_t* x, RowMap rm, const Grouping& g, int64_t n_routes,
                         int E, const tfm_affine& gate, const tfm_affine& up, int N, int Kin,
                         int bits, bool f16, uint16_t* h, hipStream_t s) {
  if (n_routes <= 0) return;
  check_shapes(N, Kin, bits, rm.nx);
  GgArgs a{};
  a.x = x; a.x_bytes = (uint32_t)(rm.nx * Kin * 2); a.rm = rm; a.g = g; a.wa = gate; a.wb = up;
  a.N = N; a.Kin = Kin; a.out = h;
  launch_mode<kGgGateUp>(a, bits, f16, n_routes, E, s);
  check_hip(hipGetLastError(), "grouped GEMM gate/up launch");
}

void launch_ggemm_down(const uint16_t* hsorted, const Grouping& g, int64_t n_routes, int E,
                       const tfm_affine& w, int N, int Kin, int bits, bool f16, uint16_t* y_sorted,
                       hipStream_t s) {
  if (n_routes <= 0) return;
  check_shapes(N, Kin, bits, n_routes);
  GgArgs a{};
  a.x = hsorted; a.x_bytes = (uint32_t)(n_routes * Kin * 2);
  a.rm = RowMap{g.order, nullptr, 1, 0, nullptr}; a.g = g; a.wa = w; a.wb = w; a.N = N;
  a.Kin = Kin; a.out = y_sorted;
  launch_mode<kGgDown>(a, bits, f16, n_routes, E, s);
  check_hip(hipGetLastError(), "grouped GEMM down launch");
}

void launch_ggemm_plain(const uint16_t* x, RowMap rm, const Grouping& g, int64_t n_routes,
                        int E, const tfm_affine& w, int N, int Kin, int bits, bool f16, uint16_t* out,
                        hipStream_t s) {
  if (n_routes <= 0) return;
  check_shapes(N, Kin, bits, rm.nx);
  GgArgs a{};
  a.x = x; a.x_bytes = (uint32_t)(rm.nx * Kin * 2); a.rm = rm; a.g = g; a.wa = w; a.wb = w;
  a.N = N; a.Kin = Kin; a.out = out;
  launch_mode<kGgPlain>(a, bits, f16, n_routes, E, s);
  check_hip(hipGetLastError(), "grouped GEMM plain launch");
}

}  // namespace tfm
