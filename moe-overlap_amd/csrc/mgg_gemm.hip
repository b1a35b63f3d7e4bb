// Persistent expert-grouped GEMM for gfx950 (MI355X).
//
// One workgroup of 256 threads (4 wave64s) per CU walks a queue of
// BLOCK_M x BLOCK_N output tiles (expert-major, then tile_m, then tile_n, the
// order of src/triton_grouped_gemm.py:277-292).  Workers either stride over
// the queue (the striped kernel, :101-154) or dequeue with a global atomic
// (:157-233).  A tile is C[off_e + tm*BM + i, tn*BN + j] = sum_k
// A[off_e + tm*BM + i, k] * B[e, k, tn*BN + j] (:36-98): rows past the expert's
// count are never stored, fp32 accumulation, output rounded to the input type.
//
// Data path per 64-wide K stage:
//   * A [BM x 64] moves HBM -> registers with 16-byte loads (8 lanes cover one
//     128-byte row segment) and is written to LDS row-major, K contiguous.
//   * B is stored [K, N] with N contiguous, but the MFMA wants 8 consecutive K
//     per lane.  Each thread loads an 8(k) x 8(n) block with eight 16-byte
//     loads (8 lanes cover 128 contiguous bytes of one row), transposes it in
//     registers with 32 v_perm_b32, and writes eight 16-byte K-contiguous
//     column segments: LDS holds B^T [BN x 64].
//   * LDS rows hold 128 bytes at a 144-byte pitch, so 16 consecutive rows read
//     at one chunk hit 16 distinct bank groups (no conflicts for the fragment
//     reads or the stores) and every LDS address is a base plus an immediate.
//   * Two LDS stages (2 x (BM + BN) x 144 B, 144 KiB at 256 x 256): the global
//     loads of stage k+1 are in flight while stage k feeds the MFMAs; one
//     barrier per stage.
//   * Waves form a 2 x 2 grid; each owns a (BM/2) x (BN/2) sub-tile made of
//     32 x 32 blocks computed with v_mfma_f32_32x32x16_{bf16,f16}.  The MFMA
//     computes C^T = B^T A^T (B^T fragment as the first operand) so each lane
//     ends up with 4 consecutive N values of one row per accumulator group,
//     stored as one 8-byte write.
#include "mgg.h"
#include "mgg_internal.h"

namespace mgg {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int kThreads = 256;
constexpr int kBK = 64;                 // K elements per LDS stage
constexpr int kLdsRow = kBK * 2 + 16;   // LDS row pitch: 8 chunks of 16 bytes + 16 pad

struct Bf16 {
  static __device__ __forceinline__ f32x16 mfma(u32x4 a, u32x4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  }
  static __device__ __forceinline__ uint32_t pack(float lo, float hi) {
    bf16x2 v = {(__bf16)lo, (__bf16)hi};
    return __builtin_bit_cast(uint32_t, v);
  }
};

struct F16 {
  static __device__ __forceinline__ f32x16 mfma(u32x4 a, u32x4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
  static __device__ __forceinline__ uint32_t pack(float lo, float hi) {
    f16x2 v = {(_Float16)lo, (_Float16)hi};
    return __builtin_bit_cast(uint32_t, v);
  }
};

// Byte offset of 16-byte chunk `chunk` (0..7) of LDS row `row`.  The 144-byte
// pitch (9 x 16 bytes, 9 odd) maps 16 consecutive rows at one chunk onto 16
// distinct 16-byte bank groups, and keeps every address base + immediate.
__device__ __forceinline__ int lds_off(int row, int chunk) { return row * kLdsRow + chunk * 16; }

__device__ __forceinline__ u32x4 lds_load(const uint8_t* base, int off) {
  return *reinterpret_cast<const u32x4*>(base + off);
}
__device__ __forceinline__ void lds_store(uint8_t* base, int off, u32x4 v) {
  *reinterpret_cast<u32x4*>(base + off) = v;
}
// Raw (unswizzled, stride 0) buffer descriptor over `bytes` bytes at `base`;
// word 3 is the gfx9-family default format.  Larger ranges are clamped to the
// 32-bit record count: in-tile offsets are far below it.
constexpr uint32_t kOutOfRange = 0x80000000u;  // any offset >= the record count
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, int64_t bytes) {
  const int64_t cap = 0x7FFFFFF0LL;
  const int32_t n = (int32_t)(bytes < 0 ? 0 : (bytes > cap ? cap : bytes));
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, n, 0x00020000);
}
__device__ __forceinline__ u32x4 bload(__amdgpu_buffer_rsrc_t rsrc, uint32_t voff, int soff) {
  return __builtin_bit_cast(u32x4,
                            __builtin_amdgcn_raw_buffer_load_b128(rsrc, (int)voff, soff, 0));
}

// Per-expert tile prefix of the derived queue, built in LDS by the whole
// workgroup: prefix[e] = sum_{j<e} ceil(max(off[j+1]-off[j],0)/BM) * n_tiles.
// Returns the queue length W = prefix[E].  Same counts as
// src/triton_grouped_gemm.py:253-271.
template <int BM>
__device__ int32_t derive_prefix(const GemmParams& p, int n_tiles, int32_t* s_prefix,
                                 int32_t* s_scan) {
  const int tid = threadIdx.x;
  const int E = p.num_experts;
  const int per = (E + kThreads - 1) / kThreads;
  const int e0 = tid * per;
  int32_t local = 0;
  for (int i = 0; i < per; ++i) {
    const int e = e0 + i;
    if (e < E) {
      const int64_t cnt = (int64_t)p.offsets[e + 1] - (int64_t)p.offsets[e];
      const int64_t tiles = cnt > 0 ? ((cnt + BM - 1) / BM) * (int64_t)n_tiles : 0;
      local += (int32_t)tiles;
    }
  }
  s_scan[tid] = local;
  __syncthreads();
  // Hillis-Steele inclusive scan over the 256 per-thread sums.
  for (int d = 1; d < kThreads; d <<= 1) {
    const int32_t add = tid >= d ? s_scan[tid - d] : 0;
    __syncthreads();
    s_scan[tid] += add;
    __syncthreads();
  }
  int32_t base = s_scan[tid] - local;
  for (int i = 0; i < per; ++i) {
    const int e = e0 + i;
    if (e < E) {
      s_prefix[e] = base;
      const int64_t cnt = (int64_t)p.offsets[e + 1] - (int64_t)p.offsets[e];
      base += cnt > 0 ? (int32_t)(((cnt + BM - 1) / BM) * (int64_t)n_tiles) : 0;
    }
  }
  if (tid == kThreads - 1) s_prefix[E] = s_scan[kThreads - 1];
  __syncthreads();
  return s_prefix[E];
}

// Cooperative zero fill of C[M, N] (the empty-queue case, :369-371).
__device__ void zero_fill(const GemmParams& p) {
  const int64_t chunks_per_row = p.n / 8;
  const int64_t total = p.m * chunks_per_row;
  const int64_t stride = (int64_t)gridDim.x * kThreads;
  const u32x4 z = {0u, 0u, 0u, 0u};
  for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < total; i += stride) {
    const int64_t r = i / chunks_per_row;
    const int64_t c8 = i - r * chunks_per_row;
    *reinterpret_cast<u32x4*>(p.c + r * p.ldc + c8 * 8) = z;
  }
}

// Computes one output tile.  All arguments are uniform across the workgroup,
// so the early returns never split a barrier.
template <int BM, int BN, class T>
__device__ __forceinline__ void run_tile(const GemmParams& p, int32_t item, int n_tiles,
                                         const int32_t* s_prefix, uint8_t* lds_a,
                                         uint8_t* lds_b) {
  constexpr int kMB = BM / 64;                 // 32-row MFMA blocks per wave
  constexpr int kNB = BN / 64;                 // 32-col MFMA blocks per wave
  constexpr int kAChunks = BM * 8 / kThreads;  // 16-byte A chunks per thread per stage
  constexpr int kARowsPerPass = kThreads / 8;  // A rows covered by one pass of the block
  constexpr int kBRows = BN / 32;              // K rows of B per thread per stage
  constexpr int kKGroups = kBK / kBRows;       // threads along K in the B load

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave & 1;
  const int wn = wave >> 1;

  int e, tm, tn;
  if (p.num_work >= 0) {
    e = p.q_expert[item];
    tm = p.q_tile_m[item];
    tn = p.q_tile_n[item];
    if ((uint32_t)e >= (uint32_t)p.num_experts || tm < 0 || (uint32_t)tn >= (uint32_t)n_tiles)
      return;
  } else {
    int lo = 0, hi = p.num_experts - 1;
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (s_prefix[mid] <= item) lo = mid; else hi = mid - 1;
    }
    e = lo;
    const int32_t local = item - s_prefix[e];
    tm = local / n_tiles;
    tn = local - tm * n_tiles;
  }

  const int64_t row0 = p.offsets[e];
  const int64_t cnt = (int64_t)p.offsets[e + 1] - row0;
  const int64_t m0 = (int64_t)tm * BM;
  const int64_t left = cnt - m0;
  if (left <= 0) return;
  const int rows_valid = left < BM ? (int)left : BM;
  const int64_t n0 = (int64_t)tn * BN;
  const int64_t K = p.k;
  const int64_t last_row = p.m - 1;

  // ---- global sources: raw buffer descriptors (uniform, per tile) --------
  // Each descriptor ends exactly at the last element of its operand, so a
  // 16-byte load past it returns zeros: rows of A past M, rows of B past K
  // and the B columns past N of the last row.  Rows of A inside [0, M) but
  // past this expert's count load the next expert's data; their results are
  // never stored.  Offsets stay 32-bit (the host bounds lda, ldb_k).
  int64_t r0 = row0 + m0;
  r0 = r0 < 0 ? 0 : (r0 > p.m ? p.m : r0);
  const int64_t a_end = r0 < p.m ? ((p.m - 1 - r0) * p.lda + K) * 2 : 0;
  const __amdgpu_buffer_rsrc_t a_rsrc = make_rsrc(p.a + r0 * p.lda, a_end);
  const int64_t b_end = ((K - 1) * p.ldb_k + p.n - n0) * 2;
  const __amdgpu_buffer_rsrc_t b_rsrc = make_rsrc(p.b + (int64_t)e * p.ldb_e + n0, b_end);

  const int a_kc = tid & 7;  // 16-byte chunk (8 K values) this thread loads
  const uint32_t a_voff = (uint32_t)(((tid >> 3) * p.lda + a_kc * 8) * 2);
  const uint32_t a_pass = (uint32_t)(kARowsPerPass * p.lda * 2);  // bytes between passes
  // B: every thread loads a kBRows(k) x 8(n) block, kBRows = 8, 4, 2 for
  // BN = 256, 128, 64, so all 256 threads take part and no load is predicated.
  const int b_kg = tid % kKGroups;  // k group: rows kBRows*b_kg .. + kBRows-1
  const int b_ng = tid / kKGroups;  // n group: columns 8*b_ng .. +7 of the tile
  // Columns past N (edge tiles) are clamped onto column N-8: in bounds, and
  // their results are never stored.
  int64_t b_col = 8 * b_ng;
  b_col = n0 + b_col > p.n - 8 ? p.n - 8 - n0 : b_col;
  const uint32_t b_voff = (uint32_t)((kBRows * b_kg * p.ldb_k + b_col) * 2);
  const uint32_t b_row = (uint32_t)(p.ldb_k * 2);

  u32x4 a_reg[kAChunks];
  u32x4 b_reg[kBRows];

  // One global load of the next stage: l < kAChunks is A chunk l, else B row
  // l - kAChunks.  A full stage (k0 + 64 <= K) has every B row and every A
  // column in range, so the uniform stage offset rides in the SGPR offset and
  // rows of A past M fall out of range through their VGPR offset alone.  In
  // the partial last stage the whole offset goes through the VGPR, so the
  // descriptor's range check zeroes A columns and B rows at k >= K.
  auto load_one = [&](int l, int64_t k0, bool tail) {
    if (l < kAChunks) {
      if (!tail) {
        a_reg[l] = bload(a_rsrc, a_voff + l * a_pass, (int)(k0 * 2));
      } else {
        const bool in = k0 + a_kc * 8 < K;
        a_reg[l] = bload(a_rsrc, in ? a_voff + (uint32_t)(k0 * 2) + l * a_pass : kOutOfRange, 0);
      }
    } else {
      const int r = l - kAChunks;
      if (!tail) {
        b_reg[r] = bload(b_rsrc, b_voff + r * b_row, (int)((uint32_t)k0 * b_row));
      } else {
        const bool in = k0 + kBRows * b_kg + r < K;
        b_reg[r] = bload(b_rsrc, in ? b_voff + ((uint32_t)k0 + r) * b_row : kOutOfRange, 0);
      }
    }
  };

  // One LDS store of the next stage: s < kAChunks stores A chunk s; else
  // column t = s - kAChunks of this thread's B block, transposed in registers
  // (b_reg[q][t/2] holds columns t&~1, t|1 of k row q) into kBRows K values.
  auto store_one = [&](int s, int buf) {
    if (s < kAChunks) {
      lds_store(lds_a + buf * (BM * kLdsRow), lds_off((tid >> 3) + kARowsPerPass * s, a_kc),
                a_reg[s]);
      return;
    }
    const int t = s - kAChunks;
    const uint32_t sel = (t & 1) ? 0x07060302u : 0x05040100u;
    uint32_t colv[kBRows / 2];
#pragma unroll
    for (int q = 0; q < kBRows / 2; ++q)
      colv[q] = __builtin_amdgcn_perm(b_reg[2 * q + 1][t >> 1], b_reg[2 * q][t >> 1], sel);
    uint8_t* dst = lds_b + buf * (BN * kLdsRow) + (8 * b_ng + t) * kLdsRow + b_kg * kBRows * 2;
    if constexpr (kBRows == 8) {
      *reinterpret_cast<u32x4*>(dst) = u32x4{colv[0], colv[1], colv[2], colv[3]};
    } else if constexpr (kBRows == 4) {
      *reinterpret_cast<u32x2*>(dst) = u32x2{colv[0], colv[1]};
    } else {
      *reinterpret_cast<uint32_t*>(dst) = colv[0];
    }
  };

  f32x16 acc[kNB][kMB];
#pragma unroll
  for (int i = 0; i < kNB; ++i)
#pragma unroll
    for (int j = 0; j < kMB; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

  const int frag_row = lane & 31;
  const int frag_half = lane >> 5;
  const int a_row_base = wm * (BM / 2) + frag_row;
  const int b_row_base = wn * (BN / 2) + frag_row;
  u32x4 fa[2][kMB];  // A fragments of two consecutive 16-wide K steps
  u32x4 fb[2][kNB];  // B^T fragments
  auto read_frag_a = [&](int buf, int kk, int slot, int j) {
    fa[slot][j] = lds_load(lds_a + buf * (BM * kLdsRow),
                           lds_off(a_row_base + 32 * j, 2 * kk + frag_half));
  };
  auto read_frag_b = [&](int buf, int kk, int slot, int i) {
    fb[slot][i] = lds_load(lds_b + buf * (BN * kLdsRow),
                           lds_off(b_row_base + 32 * i, 2 * kk + frag_half));
  };

  // One K stage in explicit program order.  The stage's 4 K steps x 4 groups
  // each issue a quarter of the K step's MFMAs followed by (a) a quarter of
  // the next K step's fragment reads, (b) in the first 8 groups, 1/8 of the
  // next stage's global loads, (c) in the last 8 groups, 1/8 of its
  // transposes and LDS stores.  sched_barrier fences keep this order: a wave
  // issues in order, so a burst of loads would stall its MFMAs behind a full
  // memory queue, and fragment reads issued late would stall each MFMA.
  // Fragments of K step 0 must already be in fa[0]/fb[0].
  constexpr int kMfmaPerStep = kMB * kNB;
  constexpr int kLoads = kAChunks + kBRows;
  constexpr int kStores = kAChunks + 8;
  auto stage = [&](int buf, int nbuf, int64_t k0_next, bool load_next, bool tail_next) {
#pragma unroll
    for (int kk = 0; kk < kBK / 16; ++kk) {
      const int cur = kk & 1;
#pragma unroll
      for (int g = 0; g < 4; ++g) {
#pragma unroll
        for (int p = g * kMfmaPerStep / 4; p < (g + 1) * kMfmaPerStep / 4; ++p) {
          const int i = p / kMB, j = p % kMB;
          acc[i][j] = T::mfma(fb[cur][i], fa[cur][j], acc[i][j]);
        }
        if (kk + 1 < kBK / 16) {
#pragma unroll
          for (int j = g; j < kMB; j += 4) read_frag_a(buf, kk + 1, cur ^ 1, j);
#pragma unroll
          for (int i = g; i < kNB; i += 4) read_frag_b(buf, kk + 1, cur ^ 1, i);
        }
        if (load_next) {
          const int grp = kk * 4 + g;  // 0..15
          if (grp < 8) {
#pragma unroll
            for (int l = grp * kLoads / 8; l < (grp + 1) * kLoads / 8; ++l)
              load_one(l, k0_next, tail_next);
          } else {
#pragma unroll
            for (int t = (grp - 8) * kStores / 8; t < (grp - 7) * kStores / 8; ++t)
              store_one(t, nbuf);
          }
        }
        __builtin_amdgcn_sched_barrier(0);
      }
    }
  };
  auto first_frags = [&](int buf) {
#pragma unroll
    for (int j = 0; j < kMB; ++j) read_frag_a(buf, 0, 0, j);
#pragma unroll
    for (int i = 0; i < kNB; ++i) read_frag_b(buf, 0, 0, i);
  };

  // Stage pipeline: stage kt computes from LDS buffer kt&1 while the next
  // stage moves global -> registers -> LDS buffer (kt+1)&1; one barrier per
  // stage.
  const int nk = (int)((K + kBK - 1) / kBK);
  const int nk_full = (int)(K / kBK);  // stages with k0 + 64 <= K
#pragma unroll
  for (int l = 0; l < kLoads; ++l) load_one(l, 0, nk_full == 0);
  __syncthreads();  // the previous tile's waves are done with the LDS stages
#pragma unroll
  for (int t = 0; t < kStores; ++t) store_one(t, 0);
  __syncthreads();
  int kt = 0;
  for (; kt + 1 < nk_full; ++kt) {
    first_frags(kt & 1);
    stage(kt & 1, (kt + 1) & 1, (int64_t)(kt + 1) * kBK, true, false);
    __syncthreads();
  }
  if (kt + 1 < nk) {  // the partial last stage when K % 64 != 0
    first_frags(kt & 1);
    stage(kt & 1, (kt + 1) & 1, (int64_t)(kt + 1) * kBK, true, true);
    __syncthreads();
    ++kt;
  }
  if (nk > 0) {
    first_frags(kt & 1);
    stage(kt & 1, 0, 0, false, false);
  }

  // ---- epilogue: acc[i][j] register r holds D[n][m] of the 32x32 block with
  // n = 8*(r/4) + 4*(lane/32) + r%4, m = lane%32 (D = C^T).
  const int64_t c_row_base = row0 + m0;
#pragma unroll
  for (int j = 0; j < kMB; ++j) {
    const int m = wm * (BM / 2) + 32 * j + frag_row;
    const int64_t grow = c_row_base + m;
    const bool row_ok = m < rows_valid && grow >= 0 && grow <= last_row;
    uint16_t* crow = p.c + grow * p.ldc;
#pragma unroll
    for (int i = 0; i < kNB; ++i) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int64_t n = n0 + wn * (BN / 2) + 32 * i + 8 * g + 4 * frag_half;
        if (row_ok && n < p.n) {
          u32x2 v;
          v[0] = T::pack(acc[i][j][4 * g + 0], acc[i][j][4 * g + 1]);
          v[1] = T::pack(acc[i][j][4 * g + 2], acc[i][j][4 * g + 3]);
          *reinterpret_cast<u32x2*>(crow + n) = v;
        }
      }
    }
  }
}

template <int BM, int BN, class T>
__global__ __attribute__((amdgpu_flat_work_group_size(kThreads, kThreads),
                          amdgpu_waves_per_eu(1, 1))) void
grouped_gemm_kernel(GemmParams p) {
  __shared__ __attribute__((aligned(16))) uint8_t lds_a[2 * BM * kLdsRow];
  __shared__ __attribute__((aligned(16))) uint8_t lds_b[2 * BN * kLdsRow];
  __shared__ int32_t s_prefix[kMaxLdsExpertsGemm + 1];
  __shared__ int32_t s_scan[kThreads];
  __shared__ int32_t s_item;

  const int tid = threadIdx.x;
  const int G = gridDim.x;
  const int n_tiles = (int)((p.n + BN - 1) / BN);

  const int32_t W = p.num_work >= 0 ? p.num_work : derive_prefix<BM>(p, n_tiles, s_prefix, s_scan);
  if (W == 0) {
    zero_fill(p);
    return;
  }

  // XCD-aware worker numbering: workgroup b runs on XCD b % 8, so giving the
  // 8 XCDs contiguous worker ranges makes each round's consecutive queue
  // items (same expert, same tile_m) share one XCD's L2.
  int v = blockIdx.x;
  if (p.remap_xcd && (G & 7) == 0) v = (blockIdx.x & 7) * (G >> 3) + (blockIdx.x >> 3);

  // Striped: items v, v+G, v+2G, ...  Atomic: the leader thread takes the
  // next ticket from the global counter and broadcasts it through LDS.
  auto next_ticket = [&]() -> int32_t {
    if (tid == 0) s_item = atomicAdd(p.counter, 1);
    __syncthreads();
    const int32_t t = s_item;
    __syncthreads();
    return t;
  };
  int32_t w = p.atomic ? next_ticket() : v;
  while ((uint32_t)w < (uint32_t)W) {
    run_tile<BM, BN, T>(p, w, n_tiles, s_prefix, lds_a, lds_b);
    w = p.atomic ? next_ticket() : w + G;
  }
  if (!p.atomic) return;
  // Every worker has fetched its final (out-of-range) ticket before adding to
  // `done`, so the last one to arrive reads the final count (W + G when no
  // worker stops early), hands it to the caller's work_counter and returns
  // both library counters to zero for the next launch on this stream.
  if (tid == 0) {
    if (atomicAdd(p.done, 1) == G - 1) {
      const int32_t final_count = atomicExch(p.counter, 0);
      atomicExch(p.done, 0);
      if (p.report != nullptr) atomicExch(p.report, final_count);
    }
  }
}

__global__ void zero_i32_kernel(int32_t* ptr, int count) {
  for (int i = threadIdx.x; i < count; i += blockDim.x) ptr[i] = 0;
}

template <class T>
int launch_typed(int block_m, int block_n, const GemmParams& p, int workers, hipStream_t stream) {
#define MGG_CASE(BM_, BN_)                                                                  \
  if (block_m == BM_ && block_n == BN_) {                                                  \
    hipLaunchKernelGGL((grouped_gemm_kernel<BM_, BN_, T>), dim3(workers), dim3(kThreads), 0, \
                       stream, p);                                                         \
    return MGG_OK;                                                                          \
  }
  MGG_CASE(256, 256)
  MGG_CASE(256, 128)
  MGG_CASE(128, 256)
  MGG_CASE(128, 128)
  MGG_CASE(128, 64)
  MGG_CASE(64, 128)
  MGG_CASE(64, 64)
  MGG_CASE(256, 64)
  MGG_CASE(64, 256)
#undef MGG_CASE
  return set_error(MGG_ERR_UNSUPPORTED, "block_m/block_n must each be one of 64, 128, 256");
}

}  // namespace

int launch_grouped_gemm(int dtype, int block_m, int block_n, const GemmParams& p, int workers,
                        hipStream_t stream) {
  int rc;
  if (dtype == MGG_DTYPE_BF16)
    rc = launch_typed<Bf16>(block_m, block_n, p, workers, stream);
  else if (dtype == MGG_DTYPE_FP16)
    rc = launch_typed<F16>(block_m, block_n, p, workers, stream);
  else
    return set_error(MGG_ERR_UNSUPPORTED, "dtype must be MGG_DTYPE_BF16 or MGG_DTYPE_FP16");
  if (rc != MGG_OK) return rc;
  return hip_error(hipGetLastError(), "grouped_gemm_kernel launch");
}

int launch_zero_i32(int32_t* ptr, int count, hipStream_t stream) {
  hipLaunchKernelGGL(zero_i32_kernel, dim3(1), dim3(64), 0, stream, ptr, count);
  return hip_error(hipGetLastError(), "zero_i32_kernel launch");
}

}  // namespace mgg
