// Stable grouping of routes by expert, in three passes over fixed chunks:
//   1. a histogram of each chunk's expert ids (hist_kernel here, or fused
//      into the routing kernel of the prefill path),
//   2. bases_kernel: per chunk and expert, the routes of that expert in
//      earlier chunks, and the expert offsets (routes to lower experts),
//   3. scatter_kernel: each workgroup places its chunk's routes in flat order
//      (ballot-matched ranks within each wave).
// Reference: MLXNativeGraniteMoEPrefill.h:666-684 (argsort of the flat expert
// ids and its inverse); the order produced is (expert asc, flat index asc).
// Ids outside [0, E) go to a last bucket E after every valid route and set
// TFM_STATUS_BAD_EXPERT_ID; offsets[E] counts the valid routes only.
#include "tfm_device.h"
#include "tfm_internal.h"

namespace tfm {

constexpr int kScatterThreads = 256;

__device__ __forceinline__ uint64_t lanemask_lt() {
  const int lane = threadIdx.x & 63;
  return lane == 0 ? 0ull : (~0ull >> (64 - lane));
}

__device__ __forceinline__ int bucket_of(int e, int E) { return (e >= 0 && e < E) ? e : E; }

__global__ __launch_bounds__(256) void hist_kernel(const int32_t* __restrict__ ids, int64_t n,
                                                   int E, int chunk, int32_t* __restrict__ hist) {
  __shared__ int h[65];
  const int tid = threadIdx.x;
  if (tid <= E) h[tid] = 0;
  __syncthreads();
  const int64_t f0 = (int64_t)blockIdx.x * chunk;
  const int64_t f1 = min(n, f0 + chunk);
  for (int64_t f = f0 + tid; f < f1; f += 256) atomicAdd(&h[bucket_of(ids[f], E)], 1);
  __syncthreads();
  if (tid <= E) hist[(int64_t)blockIdx.x * (E + 1) + tid] = h[tid];
}

// Bucket bases of every chunk from the chunk histograms:
//   part[c][b] = sum_{c' < c} hist[c'][b]   (b in [0, E])
// plus offsets (exclusive scan of the bucket totals over the E valid
// experts), the active list and the status word. One workgroup of W waves:
// wave w owns a contiguous range of chunks, lane l buckets l and 64 + l.
// Pass 1 sums each wave's range per bucket, the per-wave sums are scanned
// over waves, pass 2 walks the range again writing running prefixes. part
// may alias hist: an entry is read and then written by the same lane.
constexpr int kBaseThreads = 1024;
constexpr int kBaseWaves = kBaseThreads / 64;

__global__ __launch_bounds__(kBaseThreads) void bases_kernel(const int32_t* hist, int nblocks, int E,
                                                             int32_t* part, int32_t* __restrict__ offsets,
                                                             int32_t* __restrict__ active,
                                                             uint32_t* __restrict__ status) {
  __shared__ int wsum[kBaseWaves][66];
  __shared__ int tot[66];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int B = E + 1;
  const bool has0 = lane < B, has1 = 64 + lane < B;
  const int cpw = (nblocks + kBaseWaves - 1) / kBaseWaves;
  const int c0 = min(nblocks, wave * cpw), c1 = min(nblocks, c0 + cpw);
  // Rows are read 16 at a time with unconditional loads (indices clamped to
  // a valid entry, the value then masked), so a wave waits for memory once
  // per 16 rows rather than once per row.
  constexpr int kBatch = 16;
  // Buffer loads: entries outside this wave's rows or buckets get an offset
  // past the buffer and read as zero.
  const __amdgpu_buffer_rsrc_t rh = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<int32_t*>(hist), (short)0, (int)((uint32_t)nblocks * B * 4), 0x00020000);
  auto batch = [&](int cb, int (&v0)[kBatch], int (&v1)[kBatch]) {
#pragma unroll
    for (int k = 0; k < kBatch; ++k) {
      const int c = cb + k;
      const uint32_t row = (uint32_t)c * B * 4;
      v0[k] = __builtin_amdgcn_raw_buffer_load_b32(rh, (has0 && c < c1) ? row + lane * 4 : 0x80000000u, 0, 0);
      v1[k] = __builtin_amdgcn_raw_buffer_load_b32(rh, (has1 && c < c1) ? row + (64 + lane) * 4 : 0x80000000u, 0, 0);
    }
  };
  int s0 = 0, s1 = 0;
  for (int cb = c0; cb < c1; cb += kBatch) {
    int v0[kBatch], v1[kBatch];
    batch(cb, v0, v1);
#pragma unroll
    for (int k = 0; k < kBatch; ++k) {
      s0 += v0[k];
      s1 += v1[k];
    }
  }
  if (has0) wsum[wave][lane] = s0;
  if (has1) wsum[wave][64 + lane] = s1;
  __syncthreads();
  if (tid < B) {
    int acc = 0;
    for (int w = 0; w < kBaseWaves; ++w) {
      const int v = wsum[w][tid];
      wsum[w][tid] = acc;
      acc += v;
    }
    tot[tid] = acc;
  }
  __syncthreads();
  if (wave == 0) {
    const int t = lane < E ? tot[lane] : 0;
    int incl = t;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      const int o = __shfl_up(incl, d, 64);
      if (lane >= d) incl += o;
    }
    const int valid = __shfl(incl, 63, 64);
    if (lane < E) offsets[lane] = incl - t;
    if (lane == 0) offsets[E] = valid;
    const uint64_t act = __ballot(lane < E && t > 0);
    if (lane < E && t > 0) active[__popcll(act & lanemask_lt())] = lane;
    if (lane == 0) {
      active[E] = __popcll(act);
      *status = tot[E] > 0 ? (uint32_t)TFM_STATUS_BAD_EXPERT_ID : 0u;
    }
  }
  int r0 = has0 ? wsum[wave][lane] : 0, r1 = has1 ? wsum[wave][64 + lane] : 0;
  for (int cb = c0; cb < c1; cb += kBatch) {
    int v0[kBatch], v1[kBatch];
    batch(cb, v0, v1);
#pragma unroll
    for (int k = 0; k < kBatch; ++k) {
      const int c = cb + k;
      if (c < c1) {
        if (has0) part[(int64_t)c * B + lane] = r0;
        if (has1) part[(int64_t)c * B + 64 + lane] = r1;
      }
      r0 += v0[k];
      r1 += v1[k];
    }
  }
}

// Places the routes of chunk blockIdx.x: position of a route = first position
// of its bucket in the chunk (offsets + part; the bad-id bucket starts after
// every valid route) + its rank among the chunk's routes of that bucket.
template <int THREADS>
__global__ __launch_bounds__(THREADS) void scatter_kernel(
    const int32_t* __restrict__ ids, int64_t n, int E, int chunk, const int32_t* __restrict__ part,
    const int32_t* __restrict__ offsets, int32_t* __restrict__ order, int32_t* __restrict__ inverse) {
  __shared__ int base[65];
  __shared__ int run[65];
  __shared__ int wcnt[THREADS / 64][65];
  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int b = blockIdx.x;
  const int B = E + 1;
  for (int i = tid; i < B; i += THREADS) {
    base[i] = part[(int64_t)b * B + i] + offsets[i < E ? i : E];
    run[i] = 0;
  }
  for (int i = tid; i < (THREADS / 64) * 65; i += THREADS) (&wcnt[0][0])[i] = 0;
  __syncthreads();

  const int64_t f0 = (int64_t)b * chunk;
  const int64_t f1 = min(n, f0 + chunk);
  for (int64_t sub = f0; sub < f1; sub += THREADS) {
    const int64_t f = sub + tid;
    const bool live = f < f1;
    const int bk = live ? bucket_of(ids[f], E) : 0;
    uint64_t match = __ballot(live);
#pragma unroll
    for (int bit = 0; bit < 7; ++bit) {
      const bool on = (bk >> bit) & 1;
      const uint64_t ones = __ballot(live && on);
      match &= on ? ones : ~ones;
    }
    const int rank_w = __popcll(match & lanemask_lt());
    if (live && rank_w == 0) wcnt[wave][bk] = __popcll(match);
    __syncthreads();
    if (live) {
      int pos = base[bk] + run[bk] + rank_w;
      for (int w = 0; w < wave; ++w) pos += wcnt[w][bk];
      order[pos] = (int32_t)f;
      inverse[f] = pos;
    }
    __syncthreads();
    for (int i = tid; i < B; i += THREADS) {
      int add = 0;
      for (int w = 0; w < THREADS / 64; ++w) {
        add += wcnt[w][i];
        wcnt[w][i] = 0;
      }
      run[i] += add;
    }
    __syncthreads();
  }
}

int group_blocks(int64_t n, int chunk) { return (int)((n + chunk - 1) / chunk); }

void launch_group_scatter(const int32_t* ids, int64_t n, int E, int chunk, int32_t* hist,
                          Grouping g, uint32_t* status, hipStream_t s) {
  const int nb = group_blocks(n, chunk);
  // The chunk bases overwrite the histograms in place.
  bases_kernel<<<1, kBaseThreads, 0, s>>>(hist, nb, E, hist, g.offsets, g.active, status);
  check_hip(hipGetLastError(), "group bases launch");
  if (nb > 0) {
    // One wave per workgroup for small chunks (the routing kernel's chunks).
    if (chunk <= 64)
      scatter_kernel<64><<<nb, 64, 0, s>>>(ids, n, E, chunk, hist, g.offsets, g.order, g.inverse);
    else
      scatter_kernel<kScatterThreads><<<nb, kScatterThreads, 0, s>>>(ids, n, E, chunk, hist, g.offsets,
                                                                    g.order, g.inverse);
    check_hip(hipGetLastError(), "group scatter launch");
  }
}

void launch_group(const int32_t* ids, int64_t n, int E, Grouping g, int32_t* hist, uint32_t* status,
                  hipStream_t s) {
  const int nb = group_blocks(n, kGroupChunk);
  if (nb > 0) {
    hist_kernel<<<nb, 256, 0, s>>>(ids, n, E, kGroupChunk, hist);
    check_hip(hipGetLastError(), "group histogram launch");
  }
  launch_group_scatter(ids, n, E, kGroupChunk, hist, g, status, s);
}

}  // namespace tfm
