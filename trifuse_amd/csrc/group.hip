// Stable grouping of routes by expert: one workgroup, LDS histogram,
// exclusive scan, then a stable scatter in chunks of 1024 routes where each
// route's rank inside its wave comes from ballot-matched lanes.
// Reference: MLXNativeGraniteMoEPrefill.h:666-684 (argsort of the flat expert
// ids and its inverse); the order produced is (expert asc, flat index asc).
#include "tfm_device.h"
#include "tfm_internal.h"

namespace tfm {

constexpr int kGroupThreads = 1024;
constexpr int kGroupWaves = kGroupThreads / 64;
constexpr int kMaxBuckets = 65;  // E <= 64 experts + one bucket for bad ids

__device__ __forceinline__ uint64_t lanemask_lt() {
  const int lane = threadIdx.x & 63;
  return lane == 0 ? 0ull : (~0ull >> (64 - lane));
}

__global__ __launch_bounds__(kGroupThreads) void group_kernel(const int32_t* __restrict__ ids,
                                                              int64_t n, int E,
                                                              int32_t* __restrict__ order,
                                                              int32_t* __restrict__ inverse,
                                                              int32_t* __restrict__ offsets,
                                                              int32_t* __restrict__ active,
                                                              uint32_t* __restrict__ status,
                                                              uint32_t* __restrict__ zero,
                                                              int zero_words) {
  __shared__ int hist[kMaxBuckets];
  __shared__ int run[kMaxBuckets];
  __shared__ int wave_cnt[kGroupWaves][kMaxBuckets];
  const int tid = threadIdx.x;
  const int wv = tid >> 6;
  const int B = E + 1;  // bucket E collects out-of-range ids
  for (int i = tid; i < zero_words; i += kGroupThreads) zero[i] = 0u;
  for (int i = tid; i < B; i += kGroupThreads) hist[i] = 0;
  for (int i = tid; i < kGroupWaves * kMaxBuckets; i += kGroupThreads) (&wave_cnt[0][0])[i] = 0;
  __syncthreads();
  for (int64_t f = tid; f < n; f += kGroupThreads) {
    const int e = ids[f];
    const int b = (e >= 0 && e < E) ? e : E;
    atomicAdd(&hist[b], 1);
  }
  __syncthreads();
  if (tid == 0) {
    int acc = 0, na = 0;
    for (int b = 0; b < B; ++b) {
      run[b] = acc;
      if (b < E) {
        offsets[b] = acc;
        if (hist[b] > 0) active[na++] = b;
      }
      acc += hist[b];
    }
    offsets[E] = run[E];  // number of valid routes
    active[E] = na;
    // The grouping is the first kernel of every call that reads routes: it
    // starts the call's status word afresh.
    *status = hist[E] > 0 ? (uint32_t)TFM_STATUS_BAD_EXPERT_ID : 0u;
  }
  __syncthreads();
  // Bits needed to tell buckets 0..E apart.
  int nbits = 1;
  while ((1 << nbits) < B) ++nbits;
  for (int64_t base = 0; base < n; base += kGroupThreads) {
    const int64_t f = base + tid;
    const bool live = f < n;
    int b = 0;
    if (live) {
      const int e = ids[f];
      b = (e >= 0 && e < E) ? e : E;
    }
    // Lanes of this wave holding the same bucket.
    uint64_t match = __ballot(live);
    for (int k = 0; k < nbits; ++k) {
      const bool bit = (b >> k) & 1;
      const uint64_t ones = __ballot(live && bit);
      match &= bit ? ones : ~ones;
    }
    const int rank_in_wave = __popcll(match & lanemask_lt());
    if (live && rank_in_wave == 0) wave_cnt[wv][b] = __popcll(match);
    __syncthreads();
    if (live) {
      int pos = run[b] + rank_in_wave;
      for (int w = 0; w < wv; ++w) pos += wave_cnt[w][b];
      order[pos] = (int32_t)f;
      inverse[f] = pos;
    }
    __syncthreads();
    for (int i = tid; i < B; i += kGroupThreads) {
      int add = 0;
      for (int w = 0; w < kGroupWaves; ++w) {
        add += wave_cnt[w][i];
        wave_cnt[w][i] = 0;
      }
      run[i] += add;
    }
    __syncthreads();
  }
}

void launch_group(const int32_t* ids, int64_t n, int E, Grouping g, uint32_t* status,
                  hipStream_t s, uint32_t* zero, int zero_words) {
  group_kernel<<<1, kGroupThreads, 0, s>>>(ids, n, E, g.order, g.inverse, g.offsets, g.active,
                                           status, zero, zero_words);
  check_hip(hipGetLastError(), "group launch");
}

}  // namespace tfm
