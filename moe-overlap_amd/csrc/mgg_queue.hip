// Device-side builders for the grouped GEMM's integer metadata:
//   * expert offsets from per-expert counts
//     (expert_offsets_from_recv_counts, src/triton_grouped_gemm.py:300-323);
//   * the (expert, tile_m, tile_n) work queue
//     (_build_work_queue, src/triton_grouped_gemm.py:240-297).
// Both are integer scans over E entries; they are latency-bound single-pass
// kernels, not throughput kernels.
#include "mgg.h"
#include "mgg_internal.h"

namespace mgg {
namespace {

constexpr int kScanThreads = 1024;

// offsets[0] = 0; offsets[i+1] = sum_{j<=i} (int32)counts[j], accumulated in
// 64-bit two's complement and narrowed to Out (a wrap modulo 2^32 for int32,
// which is what cumsum-in-int64 followed by .to(int32) produces).
template <class In, class Out>
__global__ void __launch_bounds__(kScanThreads) offsets_kernel(const In* counts, int64_t E,
                                                               Out* offsets) {
  __shared__ uint64_t s_scan[kScanThreads];
  const int tid = threadIdx.x;
  const int64_t per = (E + kScanThreads - 1) / kScanThreads;
  const int64_t e0 = tid * per;
  uint64_t local = 0;
  for (int64_t i = 0; i < per; ++i) {
    const int64_t e = e0 + i;
    if (e < E) local += (uint64_t)(int64_t)(int32_t)counts[e];
  }
  s_scan[tid] = local;
  __syncthreads();
  for (int d = 1; d < kScanThreads; d <<= 1) {
    const uint64_t add = tid >= d ? s_scan[tid - d] : 0;
    __syncthreads();
    s_scan[tid] += add;
    __syncthreads();
  }
  uint64_t run = s_scan[tid] - local;
  for (int64_t i = 0; i < per; ++i) {
    const int64_t e = e0 + i;
    if (e < E) {
      run += (uint64_t)(int64_t)(int32_t)counts[e];
      offsets[e + 1] = (Out)(int64_t)run;
    }
  }
  if (tid == 0) offsets[0] = 0;
}

constexpr int kQueueThreads = 256;

// Each workgroup rebuilds the per-expert tile prefix in LDS, then writes its
// grid-stride share of the queue: item w belongs to the last expert e with
// prefix[e] <= w, at local index w - prefix[e] = tm * n_tiles + tn.
__global__ void __launch_bounds__(kQueueThreads)
queue_kernel(const int32_t* offsets, int32_t E, int32_t n_tiles, int32_t block_m, int32_t* we,
             int32_t* wm, int32_t* wn, int32_t W) {
  __shared__ int32_t s_prefix[kMaxLdsExpertsQueue + 1];
  __shared__ int32_t s_scan[kQueueThreads];
  const int tid = threadIdx.x;
  const int per = (E + kQueueThreads - 1) / kQueueThreads;
  const int e0 = tid * per;
  auto tiles_of = [&](int e) -> int32_t {
    const int64_t cnt = (int64_t)offsets[e + 1] - (int64_t)offsets[e];
    return cnt > 0 ? (int32_t)(((cnt + block_m - 1) / block_m) * (int64_t)n_tiles) : 0;
  };
  int32_t local = 0;
  for (int i = 0; i < per; ++i)
    if (e0 + i < E) local += tiles_of(e0 + i);
  s_scan[tid] = local;
  __syncthreads();
  for (int d = 1; d < kQueueThreads; d <<= 1) {
    const int32_t add = tid >= d ? s_scan[tid - d] : 0;
    __syncthreads();
    s_scan[tid] += add;
    __syncthreads();
  }
  int32_t base = s_scan[tid] - local;
  for (int i = 0; i < per; ++i) {
    if (e0 + i < E) {
      s_prefix[e0 + i] = base;
      base += tiles_of(e0 + i);
    }
  }
  if (tid == kQueueThreads - 1) s_prefix[E] = s_scan[kQueueThreads - 1];
  __syncthreads();
  const int32_t total = s_prefix[E] < W ? s_prefix[E] : W;
  for (int32_t w = blockIdx.x * kQueueThreads + tid; w < total; w += gridDim.x * kQueueThreads) {
    int lo = 0, hi = E - 1;
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (s_prefix[mid] <= w) lo = mid; else hi = mid - 1;
    }
    const int32_t loc = w - s_prefix[lo];
    const int32_t tm = loc / n_tiles;
    we[w] = lo;
    wm[w] = tm;
    wn[w] = loc - tm * n_tiles;
  }
}

}  // namespace

int launch_offsets_from_counts(const void* counts, int counts_type, int64_t E, void* offsets,
                               int out_type, hipStream_t stream) {
  const dim3 grid(1), block(kScanThreads);
  if (counts_type == MGG_INT32 && out_type == MGG_INT32)
    hipLaunchKernelGGL((offsets_kernel<int32_t, int32_t>), grid, block, 0, stream,
                       (const int32_t*)counts, E, (int32_t*)offsets);
  else if (counts_type == MGG_INT64 && out_type == MGG_INT32)
    hipLaunchKernelGGL((offsets_kernel<int64_t, int32_t>), grid, block, 0, stream,
                       (const int64_t*)counts, E, (int32_t*)offsets);
  else if (counts_type == MGG_INT32 && out_type == MGG_INT64)
    hipLaunchKernelGGL((offsets_kernel<int32_t, int64_t>), grid, block, 0, stream,
                       (const int32_t*)counts, E, (int64_t*)offsets);
  else if (counts_type == MGG_INT64 && out_type == MGG_INT64)
    hipLaunchKernelGGL((offsets_kernel<int64_t, int64_t>), grid, block, 0, stream,
                       (const int64_t*)counts, E, (int64_t*)offsets);
  else
    return set_error(MGG_ERR_INVALID, "counts_type and out_type must be MGG_INT32 or MGG_INT64");
  return hip_error(hipGetLastError(), "offsets_kernel launch");
}

int launch_build_work_queue(const int32_t* offsets, int32_t E, int64_t n_size, int block_m,
                            int block_n, int32_t* we, int32_t* wm, int32_t* wn, int32_t W,
                            hipStream_t stream) {
  if (W == 0) return MGG_OK;
  const int32_t n_tiles = (int32_t)((n_size + block_n - 1) / block_n);
  int blocks = (W + kQueueThreads - 1) / kQueueThreads;
  blocks = blocks > 1024 ? 1024 : blocks;
  hipLaunchKernelGGL(queue_kernel, dim3(blocks), dim3(kQueueThreads), 0, stream, offsets, E,
                     n_tiles, block_m, we, wm, wn, W);
  return hip_error(hipGetLastError(), "queue_kernel launch");
}

}  // namespace mgg
