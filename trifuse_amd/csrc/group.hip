// Stable grouping of routes by expert, in three passes over fixed chunks:
//   1. a histogram of each chunk's expert ids (hist_kernel here, or fused
//      into the routing kernel of the prefill path),
//   2. superblock_sums_kernel: the histograms summed over superblocks of
//      kSuperChunks chunks (one wave each),
//   3. scatter_kernel: each workgroup derives its chunk's bucket bases (the
//      superblock sums before it, the chunks of its superblock before it)
//      and the expert offsets, then places its chunk's routes in flat order
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

// Superblock sums: bsum[sb][b] = sum of hist[c][b] over the kSuperChunks
// chunks of superblock sb. One wave per superblock, lane l buckets l and
// 64 + l; all rows are requested before the first is added.
constexpr int kSuperChunks = 16;

__global__ __launch_bounds__(64) void superblock_sums_kernel(const int32_t* __restrict__ hist, int nblocks,
                                                             int E, int32_t* __restrict__ bsum) {
  const int sb = blockIdx.x;
  const int lane = threadIdx.x;
  const int B = E + 1;
  const __amdgpu_buffer_rsrc_t rh = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<int32_t*>(hist), (short)0, (int)((uint32_t)nblocks * B * 4), 0x00020000);
  int v0[kSuperChunks], v1[kSuperChunks];
#pragma unroll
  for (int k = 0; k < kSuperChunks; ++k) {
    const int c = sb * kSuperChunks + k;
    const uint32_t row = (uint32_t)c * B * 4;
    v0[k] = __builtin_amdgcn_raw_buffer_load_b32(rh, (c < nblocks && lane < B) ? row + lane * 4 : 0x80000000u, 0, 0);
    v1[k] = __builtin_amdgcn_raw_buffer_load_b32(rh, (c < nblocks && 64 + lane < B) ? row + (64 + lane) * 4 : 0x80000000u, 0, 0);
  }
  int s0 = 0, s1 = 0;
#pragma unroll
  for (int k = 0; k < kSuperChunks; ++k) {
    s0 += v0[k];
    s1 += v1[k];
  }
  if (lane < B) bsum[(int64_t)sb * B + lane] = s0;
  if (64 + lane < B) bsum[(int64_t)sb * B + 64 + lane] = s1;
}

// Grouping of zero routes: offsets all zero, no active expert (the status
// word keeps its bits).
__global__ void group_empty_kernel(int E, Grouping g, uint32_t* __restrict__ status) {
  (void)status;
  const int tid = threadIdx.x;
  if (tid <= E) g.offsets[tid] = 0;
  if (tid == 0) g.active[E] = 0;
}

static void launch_group_empty(int E, Grouping g, uint32_t* status, hipStream_t s) {
  group_empty_kernel<<<1, 128, 0, s>>>(E, g, status);
  check_hip(hipGetLastError(), "group launch");
}

// Places the routes of chunk blockIdx.x: position of a route = first position
// of its bucket in the chunk (offsets + part; the bad-id bucket starts after
// every valid route) + its rank among the chunk's routes of that bucket.
template <int THREADS>
__global__ __launch_bounds__(THREADS) void scatter_kernel(
    const int32_t* __restrict__ ids, int64_t n, int E, int chunk, const int32_t* __restrict__ hist,
    const int32_t* __restrict__ bsum, int nblocks, Grouping g, uint32_t* __restrict__ status) {
  __shared__ int base[65];
  __shared__ int run[65];
  __shared__ int wcnt[THREADS / 64][65];
  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int b = blockIdx.x;
  const int B = E + 1;
  if (tid < 64) {
    // Bucket bases of this chunk: lane l holds buckets l and 64 + l. The
    // bucket totals are every superblock's sums; the routes before this chunk
    // are the superblocks before its own plus its superblock's earlier chunks.
    const int lane = tid;
    const int nsb = (nblocks + kSuperChunks - 1) / kSuperChunks;
    const int sbi = b / kSuperChunks;
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<int32_t*>(bsum), (short)0, (int)((uint32_t)nsb * B * 4), 0x00020000);
    const __amdgpu_buffer_rsrc_t rh = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<int32_t*>(hist), (short)0, (int)((uint32_t)nblocks * B * 4), 0x00020000);
    int tot0 = 0, tot1 = 0, pre0 = 0, pre1 = 0;
    constexpr int kBatch = 32;
    // One superblock (bsum null): the totals are its own chunks' sums.
    const int nsb_sums = bsum ? nsb : 0;
    for (int r0 = 0; r0 < nsb_sums; r0 += kBatch) {
      int v0[kBatch], v1[kBatch];
#pragma unroll
      for (int k = 0; k < kBatch; ++k) {
        const int r = r0 + k;
        const uint32_t row = (uint32_t)r * B * 4;
        v0[k] = __builtin_amdgcn_raw_buffer_load_b32(rs, (r < nsb && lane < B) ? row + lane * 4 : 0x80000000u, 0, 0);
        v1[k] = __builtin_amdgcn_raw_buffer_load_b32(rs, (r < nsb && 64 + lane < B) ? row + (64 + lane) * 4 : 0x80000000u, 0, 0);
      }
#pragma unroll
      for (int k = 0; k < kBatch; ++k) {
        tot0 += v0[k];
        tot1 += v1[k];
        if (r0 + k < sbi) {
          pre0 += v0[k];
          pre1 += v1[k];
        }
      }
    }
    {
      int v0[kSuperChunks], v1[kSuperChunks];
#pragma unroll
      for (int k = 0; k < kSuperChunks; ++k) {
        const int c = sbi * kSuperChunks + k;
        const uint32_t row = (uint32_t)c * B * 4;
        const int cend = bsum ? b : nblocks;  // one superblock: every chunk, for the totals
        v0[k] = __builtin_amdgcn_raw_buffer_load_b32(rh, (c < cend && lane < B) ? row + lane * 4 : 0x80000000u, 0, 0);
        v1[k] = __builtin_amdgcn_raw_buffer_load_b32(rh, (c < cend && 64 + lane < B) ? row + (64 + lane) * 4 : 0x80000000u, 0, 0);
      }
#pragma unroll
      for (int k = 0; k < kSuperChunks; ++k) {
        const bool before = sbi * kSuperChunks + k < b;
        pre0 += before ? v0[k] : 0;
        pre1 += before ? v1[k] : 0;
        if (!bsum) {
          tot0 += v0[k];
          tot1 += v1[k];
        }
      }
    }
    // Offsets: exclusive scan of the valid experts' totals.
    const int t = lane < E ? tot0 : 0;
    int incl = t;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      const int o = __shfl_up(incl, d, 64);
      if (lane >= d) incl += o;
    }
    const int valid = __shfl(incl, 63, 64);
    if (lane < E) base[lane] = incl - t + pre0;
    // The bad-id bucket E starts after every valid route.
    if (E < 64 && lane == E) base[E] = valid + pre0;
    if (E == 64 && lane == 0) base[64] = valid + pre1;
    const int bad_total = E < 64 ? __shfl(tot0, E, 64) : __shfl(tot1, 0, 64);
    if (b == 0) {
      if (lane < E) g.offsets[lane] = incl - t;
      if (lane == 0) g.offsets[E] = valid;
      const uint64_t act = __ballot(lane < E && t > 0);
      if (lane < E && t > 0) g.active[__popcll(act & lanemask_lt())] = lane;
      if (lane == 0) {
        g.active[E] = __popcll(act);
        // Sticky: bits accumulate until tfm_status_word reads and clears them.
        if (bad_total > 0) atomicOr(status, (uint32_t)TFM_STATUS_BAD_EXPERT_ID);
      }
    }
  }
  for (int i = tid; i < B; i += THREADS) run[i] = 0;
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
      g.order[pos] = (int32_t)f;
      g.inverse[f] = pos;
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

int group_hist_rows(int64_t nblocks) {
  return (int)(nblocks + 1 + (nblocks + kSuperChunks - 1) / kSuperChunks + 1);
}

void launch_group_scatter(const int32_t* ids, int64_t n, int E, int chunk, int32_t* hist,
                          Grouping g, uint32_t* status, hipStream_t s) {
  const int nb = group_blocks(n, chunk);
  if (nb <= 0) {
    // No routes: empty offsets and active list, clear status.
    launch_group_empty(E, g, status, s);
    return;
  }
  const int nsb = (nb + kSuperChunks - 1) / kSuperChunks;
  // Superblock sums live after the chunk histograms (group_hist_rows rows).
  // With a single superblock the scatter kernel sums its chunks itself
  // (bsum null), which saves a dependent launch for small batches.
  int32_t* bsum = nullptr;
  if (nsb > 1) {
    bsum = hist + (int64_t)(nb + 1) * (E + 1);
    superblock_sums_kernel<<<nsb, 64, 0, s>>>(hist, nb, E, bsum);
    check_hip(hipGetLastError(), "group superblock sums launch");
  }
  // One wave per workgroup for small chunks (the routing kernel's chunks).
  if (chunk <= 64)
    tfm_launch(scatter_kernel<64>, nb, 64, 0, s, ids, n, E, chunk, hist, bsum, nb, g, status);
  else
    tfm_launch(scatter_kernel<kScatterThreads>, nb, kScatterThreads, 0, s, ids, n, E, chunk, hist, bsum, nb, g, status);
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
