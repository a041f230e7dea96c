// Stable grouping of routes by expert, as two passes over fixed chunks:
//   1. a histogram of each chunk's expert ids (hist_kernel here, or fused
//      into the top-k kernel of the prefill path),
//   2. scatter_kernel: each workgroup derives the first position of every
//      expert's routes in its chunk from all chunk histograms (routes to lower
//      experts, plus routes to the same expert in earlier chunks) and places
//      its routes in flat order (ballot-matched ranks within each wave).
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

__global__ __launch_bounds__(kScatterThreads) void scatter_kernel(
    const int32_t* __restrict__ ids, int64_t n, int E, int chunk, const int32_t* __restrict__ hist,
    int nblocks, int32_t* __restrict__ order, int32_t* __restrict__ inverse,
    int32_t* __restrict__ offsets, int32_t* __restrict__ active, uint32_t* __restrict__ status) {
  __shared__ int base[65];
  __shared__ int run[65];
  __shared__ int wcnt[kScatterThreads / 64][65];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int b = blockIdx.x;
  const int B = E + 1;

  // Bucket bases of this chunk: every wave sums a quarter of the chunk
  // histograms (rows c = wave mod 4) per bucket, then wave 0 combines them.
  __shared__ int part_tot[kScatterThreads / 64][65];
  __shared__ int part_pre[kScatterThreads / 64][65];
  {
    int tot = 0, pre = 0, btot = 0, bpre = 0;
    for (int c = wave; c < nblocks; c += kScatterThreads / 64) {
      if (lane < E) {
        const int v = hist[(int64_t)c * B + lane];
        tot += v;
        if (c < b) pre += v;
      }
      if (lane == 0) {
        const int v = hist[(int64_t)c * B + E];
        btot += v;
        if (c < b) bpre += v;
      }
    }
    part_tot[wave][lane] = tot;
    part_pre[wave][lane] = pre;
    if (lane == 0) {
      part_tot[wave][64] = btot;
      part_pre[wave][64] = bpre;
    }
  }
  __syncthreads();
  if (wave == 0) {
    int tot = 0, pre = 0;
#pragma unroll
    for (int w = 0; w < kScatterThreads / 64; ++w) {
      tot += part_tot[w][lane];
      pre += part_pre[w][lane];
    }
    int incl = tot;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      const int o = __shfl_up(incl, d, 64);
      if (lane >= d) incl += o;
    }
    const int excl = incl - tot;
    const int valid = __shfl(incl, 63, 64);
    if (lane < E) base[lane] = excl + pre;
    if (b == 0) {
      if (lane < E) offsets[lane] = excl;
      if (lane == 0) offsets[E] = valid;
      const uint64_t act = __ballot(lane < E && tot > 0);
      if (lane < E && tot > 0) active[__popcll(act & lanemask_lt())] = lane;
      if (lane == 0) active[E] = __popcll(act);
    }
    if (lane == 0) {
      int btot = 0, bpre = 0;
      for (int w = 0; w < kScatterThreads / 64; ++w) {
        btot += part_tot[w][64];
        bpre += part_pre[w][64];
      }
      // The bad-id bucket starts after every valid route.
      base[E] = valid + bpre;
      if (b == 0) *status = btot > 0 ? (uint32_t)TFM_STATUS_BAD_EXPERT_ID : 0u;
    }
  }
  for (int i = tid; i < (kScatterThreads / 64) * 65; i += kScatterThreads) (&wcnt[0][0])[i] = 0;
  if (tid < B) run[tid] = 0;
  __syncthreads();

  const int64_t f0 = (int64_t)b * chunk;
  const int64_t f1 = min(n, f0 + chunk);
  for (int64_t sub = f0; sub < f1; sub += kScatterThreads) {
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
    for (int i = tid; i < B; i += kScatterThreads) {
      int add = 0;
      for (int w = 0; w < kScatterThreads / 64; ++w) {
        add += wcnt[w][i];
        wcnt[w][i] = 0;
      }
      run[i] += add;
    }
    __syncthreads();
  }
}

int group_blocks(int64_t n, int chunk) { return (int)((n + chunk - 1) / chunk); }

void launch_group_scatter(const int32_t* ids, int64_t n, int E, int chunk, const int32_t* hist,
                          Grouping g, uint32_t* status, hipStream_t s) {
  const int nb = group_blocks(n, chunk);
  if (nb <= 0) {
    // No routes: offsets and the active list are all zero.
    scatter_kernel<<<1, kScatterThreads, 0, s>>>(ids, 0, E, chunk, hist, 0, g.order, g.inverse,
                                                 g.offsets, g.active, status);
  } else {
    scatter_kernel<<<nb, kScatterThreads, 0, s>>>(ids, n, E, chunk, hist, nb, g.order, g.inverse,
                                                  g.offsets, g.active, status);
  }
  check_hip(hipGetLastError(), "group scatter launch");
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
