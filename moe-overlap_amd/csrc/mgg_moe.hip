// Token <-> expert-row movement around the grouped GEMM (one GPU's share):
//   * dispatch layout: per-expert counts, offsets and a stable position for
//     every (token, slot) assignment in the expert-major row order.  This is
//     what the reference builds with sort / bincount / cumsum / inv_perm
//     (src/train_moe_baseline.py:219-237) and what DeepEP's layout kernel
//     counts per expert (third-party DeepEP csrc/kernels/layout.cu:10-121);
//   * row gather into that order (train:224, grouped_tokens = tokens[perm]);
//   * gate-weighted combine back to token order (train:246 + :340-341,
//     out += y[inv_perm] * gate, summed over the top-k slots).
// All are integer / byte-movement kernels: the layout kernels are latency
// bound, gather and combine are HBM bound.
#include "mgg.h"
#include "mgg_internal.h"

namespace mgg {
namespace {

constexpr int kLayoutThreads = 256;

// Pass 1: per-chunk expert histogram (LDS atomics), one row of `hist` per
// chunk of kLayoutChunk consecutive assignments.
template <class In>
__global__ void __launch_bounds__(kLayoutThreads)
layout_count_kernel(const In* idx, int64_t A, int32_t E, int32_t* hist) {
  extern __shared__ int32_t s_h[];
  const int tid = threadIdx.x;
  for (int e = tid; e < E; e += kLayoutThreads) s_h[e] = 0;
  __syncthreads();
  const int64_t a0 = (int64_t)blockIdx.x * kLayoutChunk;
  for (int i = tid; i < kLayoutChunk; i += kLayoutThreads) {
    const int64_t a = a0 + i;
    if (a < A) {
      const int64_t e = (int64_t)idx[a];
      if (e >= 0 && e < E) atomicAdd(&s_h[e], 1);
    }
  }
  __syncthreads();
  for (int e = tid; e < E; e += kLayoutThreads) hist[(int64_t)blockIdx.x * E + e] = s_h[e];
}

constexpr int kLayoutScanThreads = 1024;

// Pass 2 (one workgroup): offsets[e] = sum of counts of experts below e;
// hist[b][e] becomes the first position of chunk b's assignments to e
// (offsets[e] + those of chunks before b), counts[e] the total.  Threads are
// (part, expert) pairs: with fewer than 1024 experts the chunks of an expert
// are cut into `parts` ranges summed in parallel, then prefixed in LDS.
// Loads go out eight chunks at a time.
__global__ void __launch_bounds__(kLayoutScanThreads)
layout_scan_kernel(int32_t* hist, int32_t nb, int32_t E, int32_t* counts, int32_t* offsets) {
  __shared__ int32_t s_scan[kLayoutScanThreads];
  __shared__ int32_t s_part[kLayoutScanThreads];  // [parts][E] range sums, then range bases
  const int tid = threadIdx.x;
  int parts = E > 0 && E < kLayoutScanThreads ? kLayoutScanThreads / E : 1;
  parts = parts < nb ? parts : (nb > 0 ? nb : 1);
  const int per = (E + kLayoutScanThreads - 1) / kLayoutScanThreads;  // experts per thread
  auto chunk_range = [&](int part, int& b0, int& b1) {
    b0 = (int)((int64_t)part * nb / parts);
    b1 = (int)((int64_t)(part + 1) * nb / parts);
  };
  // Sum (or, with base >= 0, exclusive-prefix in place from base) chunks
  // [b0, b1) of expert e.
  auto walk = [&](int e, int b0, int b1, int32_t base) -> int32_t {
    int32_t run = base < 0 ? 0 : base;
    for (int b = b0; b < b1; b += 8) {
      int32_t c[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) c[j] = b + j < b1 ? hist[(int64_t)(b + j) * E + e] : 0;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        if (b + j < b1) {
          if (base >= 0) hist[(int64_t)(b + j) * E + e] = run;
          run += c[j];
        }
      }
    }
    return run;
  };
  int32_t local = 0;
  if (parts > 1) {
    const int e = tid % E, part = tid / E;
    int b0 = 0, b1 = 0;
    if (part < parts) {
      chunk_range(part, b0, b1);
      s_part[part * E + e] = walk(e, b0, b1, -1);
    }
    __syncthreads();
    if (part == 0) {
      int32_t run = 0;
      for (int q = 0; q < parts; ++q) {
        const int32_t c = s_part[q * E + e];
        s_part[q * E + e] = run;
        run += c;
      }
      counts[e] = run;
      local = run;
    }
  } else {
    for (int i = 0; i < per; ++i) {
      const int e = tid * per + i;
      if (e < E) {
        const int32_t run = walk(e, 0, nb, -1);
        counts[e] = run;
        local += run;
      }
    }
  }
  // Exclusive scan of the expert totals (thread t holds the total of its
  // experts; with parts > 1 only the part-0 threads, experts 0..E-1, do).
  s_scan[tid] = local;
  __syncthreads();
  for (int d = 1; d < kLayoutScanThreads; d <<= 1) {
    const int32_t add = tid >= d ? s_scan[tid - d] : 0;
    __syncthreads();
    s_scan[tid] += add;
    __syncthreads();
  }
  const int32_t first = s_scan[tid] - local;  // offset of this thread's first expert
  if (tid == kLayoutScanThreads - 1) offsets[E] = s_scan[kLayoutScanThreads - 1];
  if (parts > 1) {
    const int e = tid % E, part = tid / E;
    // Thread e is expert e's part-0 thread, so the experts below e sum to s_scan[e - 1].
    const int32_t off_e = e > 0 ? s_scan[e - 1] : 0;
    if (part == 0) offsets[e] = off_e;
    if (part < parts) {
      int b0 = 0, b1 = 0;
      chunk_range(part, b0, b1);
      walk(e, b0, b1, off_e + s_part[part * E + e]);
    }
  } else {
    int32_t base = first;
    for (int i = 0; i < per; ++i) {
      const int e = tid * per + i;
      if (e < E) {
        offsets[e] = base;
        walk(e, 0, nb, base);
        base += counts[e];
      }
    }
  }
}

// Pass 3 for any expert count (one wave per chunk, 64 assignments at a time
// in order): an assignment's position is its chunk's base for its expert plus
// the number of earlier assignments of the chunk to the same expert, so
// positions are stable (assignment order within each expert).  Lanes sharing
// an expert are grouped with ballots, one round per distinct expert in the 64.
template <class In>
__global__ void __launch_bounds__(64)
layout_scatter_kernel(const In* idx, int64_t A, int32_t top_k, int32_t E, const int32_t* hist,
                      int32_t* slot_pos, int32_t* token_index, int32_t* row_assign) {
  extern __shared__ int32_t s_base[];
  const int lane = threadIdx.x;
  for (int e = lane; e < E; e += 64) s_base[e] = hist[(int64_t)blockIdx.x * E + e];
  __syncthreads();
  const int64_t a0 = (int64_t)blockIdx.x * kLayoutChunk;
  for (int t0 = 0; t0 < kLayoutChunk; t0 += 64) {
    const int64_t a = a0 + t0 + lane;
    if (a0 + t0 >= A) break;  // uniform
    int32_t e = -1;
    if (a < A) {
      const int64_t v = (int64_t)idx[a];
      e = (v >= 0 && v < E) ? (int32_t)v : -1;
    }
    const bool valid = e >= 0;
    uint64_t todo = __ballot(valid);
    int32_t rank = 0;
    bool last = false;
    while (todo != 0) {
      const int leader = __builtin_ctzll(todo);
      const int32_t el = __builtin_amdgcn_readlane(e, leader);
      const bool mine = valid && e == el;
      const uint64_t m = __ballot(mine);
      if (mine) {
        rank = __builtin_popcountll(m & ((1ull << lane) - 1ull));
        last = lane == 63 - __builtin_clzll(m);
      }
      todo &= ~m;
    }
    if (valid) {
      const int32_t pos = s_base[e] + rank;
      slot_pos[a] = pos;
      token_index[pos] = (int32_t)(a / top_k);
      row_assign[pos] = (int32_t)a;
    } else if (a < A) {
      slot_pos[a] = -1;
    }
    __syncthreads();  // every lane has read its base before the bases move on
    if (valid && last) s_base[e] += rank + 1;
    __syncthreads();
  }
}

// Pass 3 for up to kMaxWideExperts experts: a chunk's kLayoutChunk
// assignments take one lane each (kLayoutChunk / 64 waves).  Each wave ranks
// its 64 assignments per expert with ballots and records its per-expert
// counts in LDS; a prefix over the waves, per expert, then gives each wave's
// base.  Positions are those of layout_scatter_kernel (assignment order
// within each expert), with every assignment in flight at once.
//
// kScan (small layouts, nb * E <= kFusedScanMax): pass 2 runs inside this
// pass instead of as its own launch.  `hist` then holds the count pass's
// per-chunk counts as they are, and every workgroup derives its chunk's base
// per expert from them: offsets[e] (an exclusive scan of the expert totals
// over the whole table) plus the counts of the chunks before its own.
// Workgroup 0 also writes counts and offsets.  The positions are the same.
constexpr int kWideWaves = kLayoutChunk / 64;
constexpr int kMaxWideExperts = 1024;  // [kWideWaves][E] int32 counters in 64 KiB of LDS
constexpr int64_t kFusedScanMax = 16384;  // table entries every workgroup reads (64 KiB)

template <class In, bool kScan>
__global__ void __launch_bounds__(kLayoutChunk)
layout_scatter_wide_kernel(const In* idx, int64_t A, int32_t top_k, int32_t E,
                           const int32_t* hist, int32_t nb, int32_t* counts, int32_t* offsets,
                           int32_t* slot_pos, int32_t* token_index, int32_t* row_assign) {
  extern __shared__ int32_t s_cnt[];  // [kWideWaves][E]: counts, then bases
  __shared__ int32_t s_base[kScan ? kMaxWideExperts : 1];  // kScan: chunk base per expert
  __shared__ int32_t s_wsum[kScan ? kWideWaves : 1];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = tid >> 6;
  if constexpr (kScan) {
    // Thread x < E: expert x's total over all chunks and over the chunks
    // before this one; then an exclusive scan of the totals (within each
    // wave by shuffles, then over the wave sums).
    int32_t total = 0, before = 0;
    if (tid < E) {
      for (int b0 = 0; b0 < nb; b0 += 8) {  // eight chunks' loads in flight at a time
        int32_t c[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) c[j] = b0 + j < nb ? hist[(int64_t)(b0 + j) * E + tid] : 0;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          if (b0 + j < (int)blockIdx.x) before += c[j];
          total += c[j];
        }
      }
    }
    int32_t incl = total;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      const int32_t y = __shfl_up(incl, d);
      if (lane >= d) incl += y;
    }
    if (lane == 63) s_wsum[w] = incl;
    __syncthreads();
    int32_t wbase = 0;
    for (int v = 0; v < w; ++v) wbase += s_wsum[v];
    const int32_t off = wbase + incl - total;  // offsets[tid]
    if (tid < E) {
      s_base[tid] = off + before;
      if (blockIdx.x == 0) {
        counts[tid] = total;
        offsets[tid] = off;
        if (tid == E - 1) offsets[E] = off + total;
      }
    }
  }
  for (int i = tid; i < kWideWaves * E; i += kLayoutChunk) s_cnt[i] = 0;
  __syncthreads();
  const int64_t a = (int64_t)blockIdx.x * kLayoutChunk + tid;
  int32_t e = -1;
  if (a < A) {
    const int64_t v = (int64_t)idx[a];
    e = (v >= 0 && v < E) ? (int32_t)v : -1;
  }
  const bool valid = e >= 0;
  uint64_t todo = __ballot(valid);
  int32_t rank = 0;
  while (todo != 0) {
    const int leader = __builtin_ctzll(todo);
    const int32_t el = __builtin_amdgcn_readlane(e, leader);
    const bool mine = valid && e == el;
    const uint64_t m = __ballot(mine);
    if (mine) rank = __builtin_popcountll(m & ((1ull << lane) - 1ull));
    if (lane == leader) s_cnt[w * E + el] = __builtin_popcountll(m);
    todo &= ~m;
  }
  __syncthreads();
  for (int x = tid; x < E; x += kLayoutChunk) {
    int32_t run = kScan ? s_base[x] : hist[(int64_t)blockIdx.x * E + x];
    for (int v = 0; v < kWideWaves; ++v) {
      const int32_t c = s_cnt[v * E + x];
      s_cnt[v * E + x] = run;
      run += c;
    }
  }
  __syncthreads();
  if (valid) {
    const int32_t pos = s_cnt[w * E + e] + rank;
    slot_pos[a] = pos;
    token_index[pos] = (int32_t)(a / top_k);
    row_assign[pos] = (int32_t)a;
  } else if (a < A) {
    slot_pos[a] = -1;
  }
}

constexpr int kRowThreads = 256;

// out[p, :] = x[token_index[p], :] for p < offsets[E] (read on the device, so
// the host never waits for the row count).  VEC: 16-byte chunks when every
// row start and the row length allow it, else one element at a time.
template <bool VEC>
__global__ void __launch_bounds__(kRowThreads)
gather_rows_kernel(const uint8_t* x, int64_t ld_x, const int32_t* token_index,
                   const int32_t* rows_ptr, int64_t rows_max, int64_t row_bytes, int elem,
                   uint8_t* out, int64_t ld_out) {
  const int64_t rows = rows_ptr != nullptr ? (int64_t)*rows_ptr : rows_max;
  const int64_t n = rows < rows_max ? rows : rows_max;
  for (int64_t p = blockIdx.x; p < n; p += gridDim.x) {
    const int64_t t = token_index[p];
    const uint8_t* src = x + t * ld_x * elem;
    uint8_t* dst = out + p * ld_out * elem;
    if (VEC) {
      for (int64_t c = threadIdx.x; c < row_bytes / 16; c += kRowThreads)
        reinterpret_cast<uint4*>(dst)[c] = reinterpret_cast<const uint4*>(src)[c];
    } else {
      for (int64_t c = threadIdx.x; c < row_bytes / 2; c += kRowThreads)
        reinterpret_cast<uint16_t*>(dst)[c] = reinterpret_cast<const uint16_t*>(src)[c];
    }
  }
}

template <class T>
struct Elem;
template <>
struct Elem<__bf16> {
  static __device__ __forceinline__ float load(uint16_t v) {
    return __uint_as_float((uint32_t)v << 16);
  }
  static __device__ __forceinline__ uint16_t store(float f) {
    return __builtin_bit_cast(uint16_t, (__bf16)f);
  }
};
template <>
struct Elem<_Float16> {
  static __device__ __forceinline__ float load(uint16_t v) {
    return (float)__builtin_bit_cast(_Float16, v);
  }
  static __device__ __forceinline__ uint16_t store(float f) {
    return __builtin_bit_cast(uint16_t, (_Float16)f);
  }
};

// out[t, :] = sum_j weight[t, j] * y[slot_pos[t, j], :] over the slots with a
// position (masked slots contribute nothing; a token with none gets zeros).
// fp32 accumulation in slot order, one rounding to the output type.  With
// GROUP > 1 the vector path loads the rows of GROUP slots before it adds any
// of them, with the non-temporal hint on y's rows (each read once) and on
// the output row: at top-6 and top-8 (H = 7168) 11-12% faster than one slot
// at a time with plain loads (5.0 against 4.5 TB/s), at top-2 (H = 2048,
// 6.1 TB/s with GROUP = 1) 9.5% slower, so the launch takes GROUP = 1 up to
// two slots per token.
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

template <class T, bool VEC, int GROUP>
__global__ void __launch_bounds__(kRowThreads)
combine_rows_kernel(const uint16_t* y, int64_t ld_y, const int32_t* slot_pos,
                    const float* weight, int64_t T_tokens, int32_t top_k, int64_t hidden,
                    uint16_t* out, int64_t ld_out) {
  for (int64_t t = blockIdx.x; t < T_tokens; t += gridDim.x) {
    uint16_t* dst = out + t * ld_out;
    if (VEC) {
      const int32_t* pos_t = slot_pos + t * top_k;
      const float* w_t = weight + t * top_k;
      for (int64_t c = threadIdx.x; c < hidden / 8; c += kRowThreads) {
        float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
        for (int j0 = 0; j0 < top_k; j0 += GROUP) {
          int32_t pos[GROUP];
          u32x4 v[GROUP];
#pragma unroll
          for (int g = 0; g < GROUP; ++g) {
            pos[g] = j0 + g < top_k ? pos_t[j0 + g] : -1;
            v[g] = u32x4{0u, 0u, 0u, 0u};
            if (pos[g] >= 0) {
              const u32x4* src = reinterpret_cast<const u32x4*>(y + (int64_t)pos[g] * ld_y) + c;
              if constexpr (GROUP > 1)
                v[g] = __builtin_nontemporal_load(src);
              else
                v[g] = *src;
            }
          }
#pragma unroll
          for (int g = 0; g < GROUP; ++g) {
            if (pos[g] < 0) continue;
            const float w = w_t[j0 + g];
#pragma unroll
            for (int q = 0; q < 4; ++q) {
              acc[2 * q] += w * Elem<T>::load((uint16_t)(v[g][q] & 0xFFFFu));
              acc[2 * q + 1] += w * Elem<T>::load((uint16_t)(v[g][q] >> 16));
            }
          }
        }
        u32x4 o;
#pragma unroll
        for (int q = 0; q < 4; ++q)
          o[q] = (uint32_t)Elem<T>::store(acc[2 * q]) |
                 ((uint32_t)Elem<T>::store(acc[2 * q + 1]) << 16);
        if constexpr (GROUP > 1)
          __builtin_nontemporal_store(o, reinterpret_cast<u32x4*>(dst) + c);
        else
          reinterpret_cast<u32x4*>(dst)[c] = o;
      }
    } else {
      for (int64_t c = threadIdx.x; c < hidden; c += kRowThreads) {
        float acc = 0.f;
        for (int j = 0; j < top_k; ++j) {
          const int32_t pos = slot_pos[t * top_k + j];
          if (pos < 0) continue;
          acc += weight[t * top_k + j] * Elem<T>::load(y[(int64_t)pos * ld_y + c]);
        }
        dst[c] = Elem<T>::store(acc);
      }
    }
  }
}

int grid_for(int64_t rows) {
  const int64_t g = rows < 1 ? 1 : rows;
  return (int)(g > 65536 ? 65536 : g);
}

}  // namespace

int64_t layout_chunks(int64_t assignments) {
  return (assignments + kLayoutChunk - 1) / kLayoutChunk;
}

int launch_dispatch_layout(const void* topk_idx, int idx_type, int64_t num_tokens, int top_k,
                           int32_t num_experts, int32_t* counts, int32_t* offsets,
                           int32_t* slot_pos, int32_t* token_index, int32_t* row_assign,
                           int32_t* hist, hipStream_t stream) {
  const int64_t A = num_tokens * top_k;
  const int64_t nb = layout_chunks(A);
  const size_t lds = (size_t)num_experts * sizeof(int32_t);
  if (nb > 0) {
    if (idx_type == MGG_INT64)
      hipLaunchKernelGGL(layout_count_kernel<int64_t>, dim3((unsigned)nb), dim3(kLayoutThreads),
                         lds, stream, (const int64_t*)topk_idx, A, num_experts, hist);
    else
      hipLaunchKernelGGL(layout_count_kernel<int32_t>, dim3((unsigned)nb), dim3(kLayoutThreads),
                         lds, stream, (const int32_t*)topk_idx, A, num_experts, hist);
    if (hipError_t err = hipGetLastError(); err != hipSuccess)
      return hip_error(err, "layout count launch");
  }
  // Small layouts scan inside the position pass (one launch fewer).
  const bool fused = nb > 0 && num_experts > 0 && num_experts <= kMaxWideExperts &&
                     nb * (int64_t)num_experts <= kFusedScanMax;
  if (!fused) {
    hipLaunchKernelGGL(layout_scan_kernel, dim3(1), dim3(kLayoutScanThreads), 0, stream, hist,
                       (int32_t)nb, num_experts, counts, offsets);
    if (hipError_t err = hipGetLastError(); err != hipSuccess)
      return hip_error(err, "layout scan launch");
  }
  if (nb > 0 && num_experts <= kMaxWideExperts) {
    const size_t wide_lds = (size_t)kWideWaves * lds;
#define MGG_WIDE(IN, SCAN)                                                                     \
  hipLaunchKernelGGL((layout_scatter_wide_kernel<IN, SCAN>), dim3((unsigned)nb),                \
                     dim3(kLayoutChunk), wide_lds, stream, (const IN*)topk_idx, A, top_k,        \
                     num_experts, hist, (int32_t)nb, counts, offsets, slot_pos, token_index,     \
                     row_assign)
    if (idx_type == MGG_INT64) {
      if (fused) MGG_WIDE(int64_t, true); else MGG_WIDE(int64_t, false);
    } else {
      if (fused) MGG_WIDE(int32_t, true); else MGG_WIDE(int32_t, false);
    }
#undef MGG_WIDE
    if (hipError_t err = hipGetLastError(); err != hipSuccess)
      return hip_error(err, "layout scatter launch");
  } else if (nb > 0) {
    if (idx_type == MGG_INT64)
      hipLaunchKernelGGL(layout_scatter_kernel<int64_t>, dim3((unsigned)nb), dim3(64), lds, stream,
                         (const int64_t*)topk_idx, A, top_k, num_experts, hist, slot_pos,
                         token_index, row_assign);
    else
      hipLaunchKernelGGL(layout_scatter_kernel<int32_t>, dim3((unsigned)nb), dim3(64), lds, stream,
                         (const int32_t*)topk_idx, A, top_k, num_experts, hist, slot_pos,
                         token_index, row_assign);
    if (hipError_t err = hipGetLastError(); err != hipSuccess)
      return hip_error(err, "layout scatter launch");
  }
  return MGG_OK;
}

int launch_gather_rows(const void* x, int64_t ld_x, const int32_t* token_index,
                       const int32_t* rows_ptr, int64_t rows_max, int64_t hidden, int elem_bytes,
                       void* out, int64_t ld_out, hipStream_t stream) {
  if (rows_max <= 0 || hidden <= 0) return MGG_OK;
  const int64_t row_bytes = hidden * elem_bytes;
  const bool vec = row_bytes % 16 == 0 && (ld_x * elem_bytes) % 16 == 0 &&
                   (ld_out * elem_bytes) % 16 == 0 && aligned16(x) && aligned16(out);
  if (vec)
    hipLaunchKernelGGL(gather_rows_kernel<true>, dim3(grid_for(rows_max)), dim3(kRowThreads), 0,
                       stream, (const uint8_t*)x, ld_x, token_index, rows_ptr, rows_max, row_bytes,
                       elem_bytes, (uint8_t*)out, ld_out);
  else
    hipLaunchKernelGGL(gather_rows_kernel<false>, dim3(grid_for(rows_max)), dim3(kRowThreads), 0,
                       stream, (const uint8_t*)x, ld_x, token_index, rows_ptr, rows_max, row_bytes,
                       elem_bytes, (uint8_t*)out, ld_out);
  if (hipError_t err = hipGetLastError(); err != hipSuccess)
    return hip_error(err, "gather launch");
  return MGG_OK;
}

namespace {
template <class T>
void launch_combine_typed(bool vec, int top_k, dim3 grid, dim3 block, hipStream_t stream,
                          const uint16_t* y, int64_t ld_y, const int32_t* slot_pos,
                          const float* weight, int64_t num_tokens, int64_t hidden, uint16_t* out,
                          int64_t ld_out) {
  if (!vec)
    hipLaunchKernelGGL((combine_rows_kernel<T, false, 1>), grid, block, 0, stream, y, ld_y,
                       slot_pos, weight, num_tokens, top_k, hidden, out, ld_out);
  else if (top_k <= 2)
    hipLaunchKernelGGL((combine_rows_kernel<T, true, 1>), grid, block, 0, stream, y, ld_y,
                       slot_pos, weight, num_tokens, top_k, hidden, out, ld_out);
  else
    hipLaunchKernelGGL((combine_rows_kernel<T, true, 4>), grid, block, 0, stream, y, ld_y,
                       slot_pos, weight, num_tokens, top_k, hidden, out, ld_out);
}
}  // namespace

int launch_combine_rows(int dtype, const void* y, int64_t ld_y, const int32_t* slot_pos,
                        const float* weight, int64_t num_tokens, int top_k, int64_t hidden,
                        void* out, int64_t ld_out, hipStream_t stream) {
  if (num_tokens <= 0 || hidden <= 0) return MGG_OK;
  const bool vec = hidden % 8 == 0 && ld_y % 8 == 0 && ld_out % 8 == 0 && aligned16(y) &&
                   aligned16(out);
  const dim3 grid(grid_for(num_tokens)), block(kRowThreads);
  const uint16_t* yy = (const uint16_t*)y;
  uint16_t* oo = (uint16_t*)out;
  if (dtype == MGG_DTYPE_BF16)
    launch_combine_typed<__bf16>(vec, top_k, grid, block, stream, yy, ld_y, slot_pos, weight,
                                 num_tokens, hidden, oo, ld_out);
  else
    launch_combine_typed<_Float16>(vec, top_k, grid, block, stream, yy, ld_y, slot_pos, weight,
                                   num_tokens, hidden, oo, ld_out);
  if (hipError_t err = hipGetLastError(); err != hipSuccess)
    return hip_error(err, "combine launch");
  return MGG_OK;
}

}  // namespace mgg
