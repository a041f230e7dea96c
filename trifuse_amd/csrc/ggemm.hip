// Prefill path: grouped GEMM over expert-contiguous routes.
//
// Each workgroup computes a BM x BN tile of one expert's output. Per K step of
// 64 (one quantisation group) it
//   * gathers BM activation rows (x rows of the routed tokens, or rows of the
//     expert-sorted SwiGLU output) into LDS as bf16,
//   * loads the packed 4-bit weight rows, dequantises them in registers
//     (s*q+b in fp32, rounded to bf16) and writes them to LDS,
//   * runs v_mfma_f32_32x32x16_bf16 on the two LDS tiles,
// double-buffered so the next step's global loads are in flight during the
// MFMAs. LDS rows are 64 bf16 (8 chunks of 16 B); chunk c of row r is stored
// at c ^ (r & 7), which makes the MFMA fragment reads conflict-free.
// Epilogues: SwiGLU (gate/up), gate-weighted scatter-add into an fp32
// accumulator or gate-weighted store into sorted rows (down), plain bf16
// scatter (gather_qmm).
#include "tfm_device.h"
#include "tfm_internal.h"

namespace tfm {

constexpr int BM = 128;
constexpr int BN = 128;  // weight rows per tile (gate/up: 64 gate + 64 up)
constexpr int BK = 64;
constexpr int kThreads = 256;

enum GgemmMode { kGgGateUp = 0, kGgDown = 1, kGgPlain = 2 };

struct GgArgs {
  const uint16_t* x;     // activations (x rows, or sorted h rows for down)
  RowMap rm;
  Grouping g;
  tfm_affine wa, wb;     // gate/up (wb unused otherwise)
  int N;                 // output columns of one matrix
  int Kin;
  const float* gates;    // down: fp32 gate per flat route (null: 1)
  int K;                 // routes per token (down, atomic mode)
  float* acc;            // down: fp32 [T, N] accumulator (atomic mode)
  float* P;              // down: fp32 [n_routes, N] (deterministic mode)
  uint16_t* out;         // gate/up: h [n_routes, N]; plain: out [rows, N]
  float* zero_buf;       // optional region zeroed by this launch
  int64_t zero_count;
};

// Row/column of accumulator element v of lane `lane` inside a 32x32 block of
// v_mfma_f32_32x32x16_bf16 (operands: lane l supplies row/column l%32 and
// k = 8*(l/32) .. 8*(l/32)+7).
__device__ __forceinline__ int acc_row(int v, int lane) { return 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3); }
__device__ __forceinline__ int acc_col(int lane) { return lane & 31; }

__device__ __forceinline__ int swz(int row, int chunk) { return row * BK + ((chunk ^ (row & 7)) << 3); }

template <int MODE>
__global__ __launch_bounds__(kThreads, 2) void ggemm_kernel(GgArgs args) {
  __shared__ __attribute__((aligned(16))) uint16_t sA[2][BM * BK];
  __shared__ __attribute__((aligned(16))) uint16_t sB[2][BN * BK];
  __shared__ int s_tiles[65];
  __shared__ int s_expert;

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int E = args.g.E;

  if (args.zero_buf) {
    const int64_t n4 = args.zero_count / 4;
    float4* z = reinterpret_cast<float4*>(args.zero_buf);
    for (int64_t i = (int64_t)blockIdx.x * kThreads + tid; i < n4; i += (int64_t)gridDim.x * kThreads)
      z[i] = make_float4(0.f, 0.f, 0.f, 0.f);
    if (blockIdx.x == 0)
      for (int64_t i = n4 * 4 + tid; i < args.zero_count; i += kThreads) args.zero_buf[i] = 0.f;
  }

  // M-tile prefix over experts.
  if (tid < 64) {
    int t = 0;
    if (tid < E) {
      const int cnt = args.g.offsets[tid + 1] - args.g.offsets[tid];
      t = (cnt + BM - 1) / BM;
    }
    // inclusive scan across the wave
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      const int o = __shfl_up(t, d, 64);
      if (lane >= d) t += o;
    }
    s_tiles[tid + 1] = t;
    if (tid == 0) s_tiles[0] = 0;
  }
  __syncthreads();
  const int NT = MODE == kGgGateUp ? (args.N + 63) / 64 : (args.N + BN - 1) / BN;
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
  const int seg0 = args.g.offsets[e], seg1 = args.g.offsets[e + 1];
  const int m0 = seg0 + (mt - s_tiles[e]) * BM;
  const int n0 = MODE == kGgGateUp ? nt * 64 : nt * BN;

  // ---- loader assignments: thread -> (row, half) ----
  const int lrow = tid >> 1, lhalf = tid & 1;
  // A row source
  const int aj = m0 + lrow;
  const bool a_ok = aj < seg1;
  int64_t a_src = 0;
  if (a_ok) {
    a_src = MODE == kGgDown ? (int64_t)aj : route_row(args.rm, aj);
  }
  const uint16_t* a_ptr = args.x + a_src * args.Kin + lhalf * 32;
  // B row source
  const tfm_affine* bm;
  int bn;
  if (MODE == kGgGateUp) {
    bm = lrow < 64 ? &args.wa : &args.wb;
    bn = n0 + (lrow & 63);
  } else {
    bm = &args.wa;
    bn = n0 + lrow;
  }
  const bool b_ok = bn < args.N;
  const int64_t b_row = (int64_t)e * args.N + (b_ok ? bn : 0);
  const uint32_t* b_q = bm->q + b_row * (args.Kin / 8) + lhalf * 4;
  const uint16_t* b_s = static_cast<const uint16_t*>(bm->scales) + b_row * (args.Kin / 64);
  const uint16_t* b_b = static_cast<const uint16_t*>(bm->biases) + b_row * (args.Kin / 64);

  const int KT = args.Kin / BK;
  uint4 ra[4];
  uint4 rb;
  uint16_t rs = 0, rbias = 0;

  auto gload = [&](int kt) {
    if (a_ok) {
      const uint4* p = reinterpret_cast<const uint4*>(a_ptr + kt * BK);
#pragma unroll
      for (int i = 0; i < 4; ++i) ra[i] = p[i];
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) ra[i] = make_uint4(0, 0, 0, 0);
    }
    if (b_ok) {
      rb = *reinterpret_cast<const uint4*>(b_q + kt * 8);
      rs = b_s[kt];
      rbias = b_b[kt];
    } else {
      rb = make_uint4(0, 0, 0, 0);
      rs = 0;
      rbias = 0;
    }
  };
  auto lstore = [&](int buf) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
      *reinterpret_cast<uint4*>(&sA[buf][swz(lrow, lhalf * 4 + i)]) = ra[i];
    const float s = bf2f(rs), b = bf2f(rbias);
    const uint32_t words[4] = {rb.x, rb.y, rb.z, rb.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float d[8];
      dequant8(words[i], s, b, d);
      uint4 pk;
      pk.x = pack_bf16x2(d[0], d[1]);
      pk.y = pack_bf16x2(d[2], d[3]);
      pk.z = pack_bf16x2(d[4], d[5]);
      pk.w = pack_bf16x2(d[6], d[7]);
      *reinterpret_cast<uint4*>(&sB[buf][swz(lrow, lhalf * 4 + i)]) = pk;
    }
  };

  // ---- wave tile ----
  const int wm = wave >> 1, wn = wave & 1;
  int brow[2];
  if (MODE == kGgGateUp) {
    brow[0] = wn * 32;        // gate columns
    brow[1] = 64 + wn * 32;   // up columns
  } else {
    brow[0] = wn * 64;
    brow[1] = wn * 64 + 32;
  }
  f32x16_t acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;

  gload(0);
  lstore(0);
  __syncthreads();
  for (int kt = 0; kt < KT; ++kt) {
    const int buf = kt & 1;
    if (kt + 1 < KT) gload(kt + 1);
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      const int kc = ks * 2 + (lane >> 5);
      bf16x8_t af[2], bfr[2];
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const int r = wm * 64 + i * 32 + (lane & 31);
        af[i] = *reinterpret_cast<const bf16x8_t*>(&sA[buf][swz(r, kc)]);
      }
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int r = brow[j] + (lane & 31);
        bfr[j] = *reinterpret_cast<const bf16x8_t*>(&sB[buf][swz(r, kc)]);
      }
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[i], bfr[j], acc[i][j], 0, 0, 0);
    }
    if (kt + 1 < KT) lstore(buf ^ 1);
    __syncthreads();
  }

  // ---- epilogue ----
  const int col = acc_col(lane);
#pragma unroll
  for (int i = 0; i < 2; ++i) {
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      const int j = m0 + wm * 64 + i * 32 + acc_row(v, lane);
      if (j >= seg1) continue;
      if (MODE == kGgGateUp) {
        const int n = n0 + wn * 32 + col;
        if (n < args.N)
          args.out[(int64_t)j * args.N + n] = f2bf(silu_mul(acc[i][0][v], acc[i][1][v]));
      } else if (MODE == kGgPlain) {
        const int64_t orow = args.rm.order[j];
#pragma unroll
        for (int b = 0; b < 2; ++b) {
          const int n = n0 + brow[b] + col;
          if (n < args.N) args.out[orow * args.N + n] = f2bf(acc[i][b][v]);
        }
      } else {
        const int f = args.g.order[j];
        const float gw = args.gates ? args.gates[f] : 1.0f;
#pragma unroll
        for (int b = 0; b < 2; ++b) {
          const int n = n0 + brow[b] + col;
          if (n >= args.N) continue;
          const float val = acc[i][b][v] * gw;
          if (args.acc)
            atomicAdd(&args.acc[(int64_t)(f / args.K) * args.N + n], val);
          else
            args.P[(int64_t)j * args.N + n] = val;
        }
      }
    }
  }
}

static unsigned grid_for(int64_t n_routes, int E, int NT) {
  const int64_t mt_max = (n_routes + BM - 1) / BM + (n_routes < E ? n_routes : E);
  int64_t total = mt_max * NT;
  // round up to a multiple of 8 so every XCD share is complete
  total = (total + 7) / 8 * 8;
  if (total < 8) total = 8;
  return (unsigned)total;
}

static void check_shapes(int N, int Kin) {
  if (Kin % BK != 0) fail(TFM_E_UNSUPPORTED, "grouped GEMM: input width must be a multiple of 64");
  if (N % 64 != 0) fail(TFM_E_UNSUPPORTED, "grouped GEMM: output width must be a multiple of 64");
}

void launch_ggemm_gateup(const uint16_t* x, RowMap rm, const Grouping& g, int64_t n_routes,
                         int E, const tfm_affine& gate, const tfm_affine& up, int N, int Kin,
                         uint16_t* h, float* zero_buf, int64_t zero_count, hipStream_t s) {
  if (n_routes <= 0) return;
  check_shapes(N, Kin);
  GgArgs a{};
  a.x = x; a.rm = rm; a.g = g; a.wa = gate; a.wb = up; a.N = N; a.Kin = Kin;
  a.out = h; a.zero_buf = zero_buf; a.zero_count = zero_count;
  ggemm_kernel<kGgGateUp><<<grid_for(n_routes, E, (N + 63) / 64), kThreads, 0, s>>>(a);
  check_hip(hipGetLastError(), "grouped GEMM gate/up launch");
}

void launch_ggemm_down(const uint16_t* hsorted, const Grouping& g, int64_t n_routes, int E,
                       const tfm_affine& w, int N, int Kin, const float* gates, int K,
                       float* acc, float* P, hipStream_t s) {
  if (n_routes <= 0) return;
  check_shapes(N, Kin);
  GgArgs a{};
  a.x = hsorted; a.rm = RowMap{g.order, nullptr, K, 0, nullptr}; a.g = g; a.wa = w; a.wb = w; a.N = N;
  a.Kin = Kin; a.gates = gates; a.K = K; a.acc = acc; a.P = P;
  ggemm_kernel<kGgDown><<<grid_for(n_routes, E, (N + BN - 1) / BN), kThreads, 0, s>>>(a);
  check_hip(hipGetLastError(), "grouped GEMM down launch");
}

void launch_ggemm_plain(const uint16_t* x, RowMap rm, const Grouping& g, int64_t n_routes,
                        int E, const tfm_affine& w, int N, int Kin, uint16_t* out,
                        hipStream_t s) {
  if (n_routes <= 0) return;
  check_shapes(N, Kin);
  GgArgs a{};
  a.x = x; a.rm = rm; a.g = g; a.wa = w; a.wb = w; a.N = N; a.Kin = Kin; a.out = out;
  ggemm_kernel<kGgPlain><<<grid_for(n_routes, E, (N + BN - 1) / BN), kThreads, 0, s>>>(a);
  check_hip(hipGetLastError(), "grouped GEMM plain launch");
}

}  // namespace tfm
