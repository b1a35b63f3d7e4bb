// Persistent expert-grouped GEMM for gfx950 (MI355X).
//
// A persistent grid (one workgroup per CU by default) walks a queue of
// BLOCK_M x BLOCK_N output tiles (expert-major, then tile_m, then tile_n, the
// order of src/triton_grouped_gemm.py:277-292).  Workers either stride over
// the queue (the striped kernel, :101-154) or dequeue with a global atomic
// (:157-233).  A tile is C[off_e + tm*BM + i, tn*BN + j] = sum_k
// A[off_e + tm*BM + i, k] * B[e, k, tn*BN + j] (:36-98): rows past the expert's
// count are never stored, fp32 accumulation, output rounded to the input type.
//
// Data path (run_worker): K advances in stages; A [BM x SBK] and B [SBK x BN]
// move HBM -> LDS by buffer DMA (16 bytes per lane, no VGPR staging), several
// stages ahead of the one being multiplied.  A fragments are 128-bit LDS reads;
// B stays N-contiguous in LDS and is read with the gfx950 transposing read
// ds_read_b64_tr_b16, so no transpose is ever done in registers.  The MFMA is
// v_mfma_f32_32x32x16_{bf16,f16} (fp8: v_mfma_f32_32x32x64_f8f6f4 with K-major
// B); it computes C^T = B^T A^T so each lane ends up with 4 consecutive N
// values of a row, and lanes l and l+32 swap halves so each stores 16 bytes.
#pragma once

#include "mgg.h"
#include "mgg_internal.h"

// 256x256 bf16/fp16 tiles: 32-deep K stages in a ring of four (128 KiB),
// three stages in flight while one is multiplied.  A ring of two 64-deep
// stages (one in flight) moves the same bytes per barrier pair but measured
// 5-7% slower: the K loop is bound by bytes in flight per CU.
#ifndef MGG_SBK256
#define MGG_SBK256 32
#define MGG_NS256 4
#endif
// K-major 16-bit B on the 256x256 tile: both operands' rows run along K, so
// 64-deep stages (full 128-byte lines for both, a ring of two) measured as
// fast as a ring of four 32-deep stages on uniform counts and 4-7% faster
// on skewed ones.
#ifndef MGG_KM_SBK256
#define MGG_KM_SBK256 64
#define MGG_KM_NS256 2
#endif
#ifndef MGG_NW256
#define MGG_NW256 8
#endif
// A in 64-deep blocks on the 256x256 16-bit tile (see ablk_mode), with a B
// ring of MGG_ABLK_BS 32-deep stages.
#ifndef MGG_ABLK
#define MGG_ABLK 1
#endif
#ifndef MGG_ABLK_BS
#define MGG_ABLK_BS 4
#endif
#ifndef MGG_FP8_NW
#define MGG_FP8_NW 8
#endif
// K loops split into stages known to lie wholly inside K (issued without the
// partial-stage checks) and the rest.
#ifndef MGG_FULL_LOOP
#define MGG_FULL_LOOP 1
#endif
// Atomic schedule with the device-derived queue: every whole round of G tiles
// by the striped placement, tickets only for the tail past them.
#ifndef MGG_STATIC_ROUNDS
#define MGG_STATIC_ROUNDS 1
#endif
// Device-derived queue: an expert's tiles in groups of MGG_GROUP_M m-tiles,
// n-tile by n-tile inside a group (see decode).
#ifndef MGG_GROUP_M
#define MGG_GROUP_M 4
#endif
// Non-temporal B DMAs on the 128x512 tile (kBStream).
#ifndef MGG_BSTREAM
#define MGG_BSTREAM 1
#endif
// Split last round: each K part of an even cut at least this deep (a
// part's meetings cost about as much as 1024 of K on the 256x256 tile).
#ifndef MGG_SPLIT_MIN_K
#define MGG_SPLIT_MIN_K 1024
#endif
// Split last round: K by which part q is cut shorter per bit set in q.
#ifndef MGG_SPLIT_STAGGER_K
#define MGG_SPLIT_STAGGER_K 384
#endif
// Most parts a tile of a short last round is split into.
#ifndef MGG_SPLIT_MAX
#define MGG_SPLIT_MAX 4
#endif

namespace mgg {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef int32_t i32x4 __attribute__((ext_vector_type(4)));
typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) i16x4 lds_i16x4;

typedef uint32_t u32x8 __attribute__((ext_vector_type(8)));
typedef int32_t i32x8 __attribute__((ext_vector_type(8)));

// Operand types.  kElem: bytes per element; kMfmaK: K of one 32x32 MFMA;
// Frag: one lane's operand of it (8 consecutive K of a row for 16-bit types,
// 32 for fp8); kBKMajor: B is stored [E, N, K] (K contiguous) rather than
// [E, K, N]; kScaled: the output is scaled per row of A and per (expert,
// column of B) before rounding.  The output is 16-bit in every case.
struct Bf16 {
  static constexpr int kElem = 2, kMfmaK = 16;
  static constexpr bool kBKMajor = false, kScaled = false;
  using Frag = u32x4;
  static __device__ __forceinline__ f32x16 mfma(Frag a, Frag b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  }
  static __device__ __forceinline__ uint32_t pack(float lo, float hi) {
    bf16x2 v = {(__bf16)lo, (__bf16)hi};
    return __builtin_bit_cast(uint32_t, v);
  }
  static __device__ __forceinline__ float to_float(uint16_t h) {
    return __builtin_bit_cast(float, (uint32_t)h << 16);
  }
};

struct F16 {
  static constexpr int kElem = 2, kMfmaK = 16;
  static constexpr bool kBKMajor = false, kScaled = false;
  using Frag = u32x4;
  static __device__ __forceinline__ f32x16 mfma(Frag a, Frag b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
  static __device__ __forceinline__ uint32_t pack(float lo, float hi) {
    f16x2 v = {(_Float16)lo, (_Float16)hi};
    return __builtin_bit_cast(uint32_t, v);
  }
  static __device__ __forceinline__ float to_float(uint16_t h) {
    return (float)__builtin_bit_cast(_Float16, h);
  }
};

// 16-bit operands with B stored [E, N, K]: B's tile rows are loaded like A's
// (rows of K) and its fragments are plain 16-byte row reads, which hold the
// same values per lane as the transposing reads of [E, K, N] B, so the MFMA
// sequence and the results are the same bit for bit.
struct Bf16K : Bf16 {
  static constexpr bool kBKMajor = true;
};
struct F16K : F16 {
  static constexpr bool kBKMajor = true;
};

// OCP fp8 e4m3 operands (v_mfma_f32_32x32x64_f8f6f4, both formats e4m3: lane
// l holds row l%32, K 32*(l/32) .. +31), bf16 output.  The scaled builtin with
// zero scale operands is the unscaled instruction.
struct Fp8 {
  static constexpr int kElem = 1, kMfmaK = 64;
  static constexpr bool kBKMajor = true, kScaled = true;
  using Frag = u32x8;
  static __device__ __forceinline__ f32x16 mfma(Frag a, Frag b, f32x16 c) {
    return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(
        __builtin_bit_cast(i32x8, a), __builtin_bit_cast(i32x8, b), c, 0, 0, 0, 0, 0, 0);
  }
  static __device__ __forceinline__ uint32_t pack(float lo, float hi) { return Bf16::pack(lo, hi); }
};

__device__ __forceinline__ u32x4 lds_load(const uint8_t* base, int off) {
  return *reinterpret_cast<const u32x4*>(base + off);
}
__device__ __forceinline__ __attribute__((address_space(3))) uint8_t* lds_ptr(uint8_t* p) {
  return (__attribute__((address_space(3))) uint8_t*)p;
}
// A voffset at or past every descriptor's record count (records are clamped
// below 2^31): a DMA lane given it writes zeros to LDS and reads no memory.
constexpr uint32_t kOutOfRange = 0x80000000u;

template <int V>
struct IntConst {
  static constexpr int value = V;
};

// f(IntConst<0>{}), ..., f(IntConst<N-1>{}) in order.
template <int N, int I = 0, class F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (I < N) {
    f(IntConst<I>{});
    static_for<N, I + 1>(f);
  }
}

// Fused epilogues (element-wise on the fp32 accumulator, before rounding to
// 16 bits).  They run on 128 values per lane per tile while the matrix cores
// wait, so they use the hardware reciprocal and base-2 exponential (about
// 1 ulp each) instead of the library's correctly rounded routines.
__device__ __forceinline__ float exp_neg(float x) {  // e^(-x)
  return __builtin_amdgcn_exp2f(-1.44269504088896341f * x);
}
// erf(z) for z >= 0 by Abramowitz & Stegun, Handbook of Mathematical
// Functions, formula 7.1.26: 1 - t(a1 + t(a2 + t(a3 + t(a4 + t a5)))) e^(-z^2),
// t = 1/(1 + p z), |error| <= 1.5e-7.
__device__ __forceinline__ float erf_pos(float z) {
  const float t = __builtin_amdgcn_rcpf(1.0f + 0.3275911f * z);
  const float poly =
      t * (0.254829592f + t * (-0.284496736f + t * (1.421413741f + t * (-1.453152027f + t * 1.061405429f))));
  return 1.0f - poly * exp_neg(z * z);
}
__device__ __forceinline__ float gelu_erf(float x) {  // torch.nn.functional.gelu, exact (erf) form
  const float e = erf_pos(fabsf(x) * 0.70710678118654752f);
  return 0.5f * x * (1.0f + copysignf(e, x));
}
__device__ __forceinline__ float silu_mul(float gate, float up) {  // silu(gate) * up
  // e^(-gate) overflows to inf for gate < -88: the reciprocal is then 0 and
  // so is the result, as silu's limit is.
  return gate * __builtin_amdgcn_rcpf(1.0f + exp_neg(gate)) * up;
}

// Per-expert tile prefix of the derived queue, built in LDS by the whole
// workgroup: prefix[e] = sum_{j<e} ceil(max(off[j+1]-off[j],0)/BM) * n_tiles.
// Returns the queue length W = prefix[E].  Same counts as
// src/triton_grouped_gemm.py:253-271.  With `rep_tiles` set, *w_report gets
// the queue length of the report tile (p.report_bm x p.report_bn, rep_tiles
// column tiles) from the same pass over the offsets; else it is W.
template <int BM, int NT>
__device__ int32_t derive_prefix(const GemmParams& p, int n_tiles, int32_t* s_prefix,
                                 int32_t* s_offs, int32_t* s_scan, int rep_tiles,
                                 int32_t* w_report) {
  const int tid = threadIdx.x;
  const int E = p.num_experts;
  const int per = (E + NT - 1) / NT;
  const int e0 = tid * per;
  int32_t local = 0;
  int64_t rep_local = 0;
  for (int i = 0; i < per; ++i) {
    const int e = e0 + i;
    if (e < E) {
      const int64_t cnt = (int64_t)p.offsets[e + 1] - (int64_t)p.offsets[e];
      const int64_t tiles = cnt > 0 ? ((cnt + BM - 1) / BM) * (int64_t)n_tiles : 0;
      local += (int32_t)tiles;
      if (rep_tiles > 0 && cnt > 0) rep_local += ((cnt + p.report_bm - 1) / p.report_bm) * (int64_t)rep_tiles;
    }
  }
  // Inclusive scan of the NT per-thread sums: within each wave by lane
  // shuffles, then across the NT/64 wave totals (one barrier).  The report
  // count is a plain sum (wave totals in s_scan[NT/64 ..]).
  const int lane = tid & 63;
  const int wave = tid >> 6;
  int32_t incl = local;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const int32_t y = __shfl_up(incl, d);
    if (lane >= d) incl += y;
  }
  if (rep_tiles > 0) {
    int32_t r = (int32_t)rep_local;  // the reference's int32 counter wraps the same way
#pragma unroll
    for (int d = 32; d >= 1; d >>= 1) r += __shfl_xor(r, d);
    if (lane == 0) s_scan[NT / 64 + wave] = r;
  }
  if (lane == 63) s_scan[wave] = incl;
  __syncthreads();
  if (rep_tiles > 0) {
    int32_t r = 0;
    for (int v = 0; v < NT / 64; ++v) r += s_scan[NT / 64 + v];
    *w_report = r;
  }
  for (int v = 0; v < wave; ++v) incl += s_scan[v];
  int32_t base = incl - local;
  for (int i = 0; i < per; ++i) {
    const int e = e0 + i;
    if (e < E) {
      s_prefix[e] = base;
      if (s_offs != nullptr) s_offs[e] = p.offsets[e];
      const int64_t cnt = (int64_t)p.offsets[e + 1] - (int64_t)p.offsets[e];
      base += cnt > 0 ? (int32_t)(((cnt + BM - 1) / BM) * (int64_t)n_tiles) : 0;
    }
  }
  if (tid == NT - 1) {
    s_prefix[E] = incl;
    if (s_offs != nullptr) s_offs[E] = p.offsets[E];
  }
  __syncthreads();
  const int32_t W = s_prefix[E];
  if (rep_tiles <= 0) *w_report = W;
  return W;
}

// sum_e ceil(max(off[e+1]-off[e], 0) / bm) * n_tiles over every expert (any
// count), wrapped to int32 as the reference's int32 counter wraps; the whole
// workgroup calls it.
template <int NT>
__device__ int32_t queue_length(const GemmParams& p, int bm, int n_tiles, int32_t* s_scan) {
  const int tid = threadIdx.x;
  int64_t local = 0;
  for (int e = tid; e < p.num_experts; e += NT) {
    const int64_t cnt = (int64_t)p.offsets[e + 1] - (int64_t)p.offsets[e];
    if (cnt > 0) local += ((cnt + bm - 1) / bm) * (int64_t)n_tiles;
  }
  int32_t r = (int32_t)local;
#pragma unroll
  for (int d = 32; d >= 1; d >>= 1) r += __shfl_xor(r, d);
  __syncthreads();  // s_scan may hold another reduction's values
  if ((tid & 63) == 0) s_scan[tid >> 6] = r;
  __syncthreads();
  int32_t total = 0;
  for (int v = 0; v < NT / 64; ++v) total += s_scan[v];
  __syncthreads();
  return total;
}

// Dequeue tickets of the atomic schedule come from a 64-bit word (epoch << 32)
// | count, where `epoch` is this launch's tag.  A launch that runs to its end
// leaves the word at (next_epoch << 32) | 0, next_epoch being the tag the
// host gives the next launch on the same word, so that launch's tickets are
// plain atomic adds.  A word holding another epoch (a launch that did not
// finish, a caller that overwrote the memory, a reused word) is claimed: the
// worker that finds it reads it and, unless it already carries this launch's
// epoch, swaps in (epoch, 1) and holds ticket 0; a worker that loses the
// swap to another claim takes an ordinary ticket.  Called by one lane per
// workgroup.
__device__ __forceinline__ int32_t first_ticket(unsigned long long* word, uint32_t epoch) {
  const unsigned long long tagged = ((unsigned long long)epoch << 32) | 1ull;
  unsigned long long cur = __hip_atomic_load(word, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  for (;;) {
    if ((uint32_t)(cur >> 32) == epoch) {
      const unsigned long long t = atomicAdd(word, 1ull);
      if ((uint32_t)(t >> 32) == epoch) return (int32_t)(uint32_t)t;
      cur = t + 1;  // cannot happen while one launch owns the word; claim again
      continue;
    }
    const unsigned long long seen = atomicCAS(word, cur, tagged);
    if (seen == cur) return 0;
    cur = seen;
  }
}
// The ticket held by `raw`, the value an atomic add of 1 on the word returned.
__device__ __forceinline__ int32_t ticket_from(unsigned long long raw, unsigned long long* word,
                                               uint32_t epoch) {
  if ((uint32_t)(raw >> 32) == epoch) return (int32_t)(uint32_t)raw;
  return first_ticket(word, epoch);
}

// Cooperative zero fill of C[M, cols] (the empty-queue case, :369-371): 8
// columns per lane, the last chunk of a row (cols not a multiple of 8) by
// words (cols even) or by elements (kOdd: cols odd).
template <bool kOdd>
__device__ void zero_fill(const GemmParams& p, int64_t cols) {
  const int64_t chunks_per_row = (cols + 7) / 8;
  const int64_t total = p.m * chunks_per_row;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  const u32x4 z = {0u, 0u, 0u, 0u};
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += stride) {
    const int64_t r = i / chunks_per_row;
    const int64_t c8 = i - r * chunks_per_row;
    uint16_t* dst = p.c + r * p.ldc + c8 * 8;
    if (c8 * 8 + 8 <= cols) {
      *reinterpret_cast<u32x4*>(dst) = z;
    } else if constexpr (kOdd) {
      for (int64_t j = 0; c8 * 8 + j < cols; ++j) dst[j] = 0;
    } else {
      for (int64_t w = 0; c8 * 8 + 2 * w < cols; ++w) reinterpret_cast<uint32_t*>(dst)[w] = 0u;
    }
  }
}

// One 16-byte-per-lane DMA from global memory (through a buffer descriptor)
// straight into LDS: lane l's 16 bytes land at LDS byte address
// lds + 16*l, so a wave fills 1 KiB.  Issued from inline assembly so that the
// compiler does not treat every later LDS read as dependent on it (it cannot
// tell DMA targets apart and would wait for all of them); the kernel waits
// on the DMA explicitly (wait_dma) before the barrier that publishes a stage.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void dma16(i32x4 rsrc, uint32_t voff, uint32_t soff, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %3\n\tbuffer_load_dwordx4 %0, %1, %2 offen lds"
               :
               : "v"(voff), "s"(rsrc), "s"(soff), "s"(lds)
               : "memory", "m0");
}
// The same with the non-temporal hint: for operand lines no other tile of
// the launch reads again, so they leave L2 early.
__device__ __forceinline__ void dma16_nt(i32x4 rsrc, uint32_t voff, uint32_t soff, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %3\n\tbuffer_load_dwordx4 %0, %1, %2 offen nt lds"
               :
               : "v"(voff), "s"(rsrc), "s"(soff), "s"(lds)
               : "memory", "m0");
}
// One 4-byte-per-lane DMA: lane l's word lands at LDS byte address lds + 4*l.
__device__ __forceinline__ void dma4(i32x4 rsrc, uint32_t voff, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %2\n\tbuffer_load_dword %0, %1, 0 offen lds"
               :
               : "v"(voff), "s"(rsrc), "s"(lds)
               : "memory", "m0");
}
#pragma clang diagnostic pop
// Waits until at most N of this wave's DMAs are outstanding.
template <int N>
__device__ __forceinline__ void wait_dma() {
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// Waits until at most min(later, MAXL) * D of this wave's DMAs are outstanding,
// i.e. every DMA issued before the last `later` groups of D has completed.
template <int D, int MAXL>
__device__ __forceinline__ void wait_dma_groups(int later) {
  if constexpr (MAXL > 0) {
    if (later >= MAXL) {
      wait_dma<MAXL * D>();
      return;
    }
    wait_dma_groups<D, MAXL - 1>(later);
  } else {
    wait_dma<0>();
  }
}

__device__ __forceinline__ i32x4 make_rsrc4(const void* base, int64_t bytes) {
  const int64_t cap = 0x7FFFFFF0LL;
  const uint64_t addr = reinterpret_cast<uint64_t>(base);
  i32x4 r;
  r[0] = __builtin_amdgcn_readfirstlane((int32_t)(uint32_t)addr);
  r[1] = __builtin_amdgcn_readfirstlane((int32_t)(uint32_t)((addr >> 32) & 0xFFFFu));  // stride 0
  r[2] = __builtin_amdgcn_readfirstlane((int32_t)(bytes < 0 ? 0 : (bytes > cap ? cap : bytes)));
  r[3] = 0x00020000;  // gfx9-family default format
  return r;
}

__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}

// A in blocks of two stages: the 256x256 16-bit N-major tile with 32-deep
// stages loads A in 64-deep blocks, so each A row segment is a full 128-byte
// line (half the L2 requests of 64-byte segments), into two LDS slots of
// 32 KiB, while B keeps 32-deep stages in a ring of MGG_ABLK_BS slots.
template <int BM, int BN, int SBK, int NSTAGE, int NW, class T>
constexpr bool ablk_mode() {
  return MGG_ABLK && BM == 256 && BN == 256 && SBK == 32 && NSTAGE == 4 && NW == 8 &&
         T::kElem == 2 && !T::kBKMajor && !T::kScaled;
}

// One workgroup's share of the queue: a persistent loop over tiles.  All
// arguments, and every branch below that guards a barrier, are uniform across
// the workgroup.
//
// K advances in stages of SBK elements; NSTAGE stages rotate through LDS.
// A stage holds A [BM x SBK] as BM rows of SBK*kElem bytes and B [SBK x BN]
// in its global layout (K rows of BN contiguous N values; K-major fp8 B is
// stored like A); both arrive by DMA, NSTAGE-1 stages ahead of the one being
// multiplied.  16-byte chunks are
// XOR-swizzled on the global side so that the fragment reads below are
// bank-conflict free:
//   A row r, chunk c  -> physical chunk c ^ ((r >> 3) & 1)    (32-byte rows)
//                                        c ^ ((r >> 2) & 3)    (64-byte rows)
//                                        c ^ ((r >> 1) & 7)    (128-byte rows)
//   B row k, chunk c  -> physical chunk c ^ 4*(k & 3)          (BN >= 128)
//                                        c ^ 4*((k >> 1) & 1)  (BN == 64)
// A fragments are ds_read_b128 (8 consecutive K of one row).  B fragments use
// the gfx950 transposing read ds_read_b64_tr_b16: in each group of 16 lanes,
// lane s addresses B[k0 + s/4][n0 + 4*(s%4) .. +3] and lane j receives
// B[k0 .. k0+3][n0 + j], so two reads give a lane the 8 consecutive K of its
// column that the MFMA expects.
//
// Consecutive tiles overlap: once a tile's last stage has been read from LDS,
// the next tile is decoded and its first stage is issued before the finished
// tile's stores, so the next tile's first DMA latency hides behind the
// epilogue; in atomic mode the ticket of the next tile is taken early in the
// current one.  `first` is this worker's first item (a ticket in atomic mode).
template <int BM, int BN, int SBK, int NSTAGE, int NW, class T, int EPI>
__device__ __forceinline__ void run_worker(const GemmParams& p, int32_t W_tiles, int32_t w_report,
                                           int32_t first, int n_tiles,
                                           const int32_t* s_prefix,
                                           const int32_t* s_offs, int32_t* s_item, uint8_t* lds,
                                           float* s_scale) {
  constexpr int kBK = SBK;                  // K (elements) per stage
  constexpr int kStages = NSTAGE;           // LDS stages in rotation
  constexpr int kE = T::kElem;              // bytes per operand element
  constexpr int kChunkElems = 16 / kE;      // elements per 16-byte chunk
  constexpr int kSteps = kBK / T::kMfmaK;   // MFMA K steps per stage
  constexpr int kARowBytes = kBK * kE;
  constexpr int kAChunks = kARowBytes / 16; // 16-byte chunks per A row
  constexpr int kARowsPerDma = 64 / kAChunks;
  constexpr int kAStage = BM * kARowBytes;  // bytes of A per stage
  constexpr int kBStage = kBK * BN * kE;    // bytes of B per stage
  // LDS rows of B: K-major B is stored like A (BN rows of the stage's K
  // bytes); otherwise K rows of BN 16-bit values.
  constexpr int kBRowBytes = T::kBKMajor ? kARowBytes : BN * 2;
  // LDS layout of A: a stage per slot, or (kABlk) a block of two stages per
  // slot with 128-byte rows; kAPerWave counts the DMAs of one slot.
  constexpr bool kABlk = ablk_mode<BM, BN, SBK, NSTAGE, NW, T>();
  constexpr int kALdsRow = kABlk ? 2 * kARowBytes : kARowBytes;
  constexpr int kALdsChunks = kALdsRow / 16;
  constexpr int kARowsPerDmaL = 64 / kALdsChunks;
  constexpr int kASlot = BM * kALdsRow;
  constexpr int kASlots = kABlk ? 2 : kStages;
  constexpr int kBSlots = kABlk ? MGG_ABLK_BS : kStages;
  constexpr int kLB = kBSlots - 1;  // kABlk: B stages issued ahead
  static_assert(!kABlk || (kLB >= 3 && kSteps == 2), "A blocks need a B ring of 4+ and 2-step stages");
  constexpr int kAPerWave = BM / (NW * kARowsPerDmaL);  // A DMAs per wave per A slot
  constexpr int kBPerWave = kBStage / (1024 * NW);      // B DMAs per wave per stage
  constexpr int kWN = NW / 2;                          // waves along N (2 along M)
  static_assert(kAPerWave >= 1 && kBPerWave >= 1, "tile too small for the wave count");
  static_assert(kSteps == 1 || kSteps == 2 || kSteps == 4, "a stage must be 1, 2 or 4 MFMA K steps");
  static_assert(kStages >= 2, "need at least two LDS stages");
  constexpr int kDmaPerStage = kAPerWave + kBPerWave;
  constexpr int kBChunks = kBRowBytes / 16;  // 16-byte chunks per B row
  constexpr int kBRowsPerDma = 64 / kBChunks;
  // 16-byte chunks of one MFMA K step in a row, and of one lane's fragment.
  constexpr int kStepChunks = T::kMfmaK * kE / 16;
  constexpr int kFragChunks = kStepChunks / 2;
  constexpr int kMB = BM / 64;              // 32-row MFMA blocks per wave
  constexpr int kNB = BN / (32 * kWN);      // 32-col MFMA blocks per wave
  static_assert(kNB >= 1, "tile too narrow for the wave count");

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave & 1;
  const int wn = wave >> 1;
  const int G = gridDim.x;
  const int64_t K = p.k;
  // ---- split last round (atomic schedule, device-derived queue) ----------
  // When the rem tiles past the last full round of G are at most G/s for
  // some s in 2 .. MGG_SPLIT_MAX (the largest such s is taken; the library
  // provided the partial-sum workspace), each of them becomes s work items,
  // the parts q = 0 .. s-1 of K, [K_q, K_q+1) in whole granules (cut
  // unevenly, see kSplitStagger), taken by s workers: the last round runs on
  // s times as many CUs for about 1/s as long.  Queue items past w_base are
  // the parts (item w_base + s*t + q is part q of tile w_base + t); W counts
  // work items.  The parts
  // meet pairwise in split_fixup.  A granule is an A block (A-block tile) or
  // a stage, so every part starts on a stage boundary; each part holds at
  // least MGG_SPLIT_MIN_K of K in an even cut (the meetings, about 7-20 µs a tree level
  // depending on the card, outweigh shorter parts: with K = 2048 halves
  // measured 1.5-1.9% faster than quarters on the skewed workload).  The
  // striped schedule keeps whole tiles.
  constexpr int kGran = kABlk ? 2 * kBK : kBK;
  const int n_gran = (int)((K + kGran - 1) / kGran);
  // (Both in 16-bit K: fp8 parts are twice as deep, its MFMAs taking half
  // the time per K; fp8 256x128 at K = 2048 in halves ran 7.9% slower than
  // whole tiles.)
  constexpr int kMinPartGran = (MGG_SPLIT_MIN_K * 2 / kE + kGran - 1) / kGran;
  // Parts are cut unevenly: at every meeting of the tree the higher subtree
  // (the one whose parts have that level's bit set) should arrive first and
  // write its sums while the lower one still runs K steps, so that the
  // lower one only reads (parts of even length arrive together and both
  // write).  Part q gets kSplitStagger granules less per bit set in q.
  // 384 of K measured best for halves (skewed atomic -1.7 to -1.9% against
  // even halves, up GEMM -0.6%; 512 and more slower again); thirds with it,
  // the down GEMM -0.7%.
  constexpr int kSplitStagger = (MGG_SPLIT_STAGGER_K * 2 / kE + kGran - 1) / kGran;
  int32_t w_base = W_tiles;
  int32_t W = W_tiles;
  int split_s = 1;  // parts per split tile
  if (p.atomic && p.num_work < 0 && p.split_flags != nullptr) {
    const int32_t rem = W_tiles > G ? W_tiles % G : W_tiles;
    for (int sp = MGG_SPLIT_MAX; sp >= 2 && split_s == 1; --sp)
      if (rem > 0 && (int64_t)rem * sp <= G && (int64_t)rem * sp <= p.split_slots && n_gran >= kMinPartGran * sp)
        split_s = sp;
    if (split_s > 1) {
      w_base = W_tiles - rem;
      W = w_base + rem * split_s;
    }
  }
  // Atomic schedule: a worker's first S items are its stripes (items v, v+G,
  // ..., in the striped schedule's XCD-aware placement, no ticket), the rest
  // go by tickets t of the global counter, standing for items S*G + t.  With
  // the queue derived on the device and at least two rounds of tiles, S is
  // the number of whole rounds (floor(W_tiles / G)): every whole round keeps
  // each XCD's L2 sharing few A and B blocks (the queue's grouped order), and
  // only the tail past them (the split parts, or whole tiles when the tail
  // is too long to split) is drawn by ticket.  Otherwise S = 1.
  // Items past S*G take one ticket each (W - S*G of them when W > S*G) and
  // every worker with a first item (min(W, G) of them) draws one ticket past
  // the queue before it stops, so the worker that draws the last ticket,
  // W - S*G + G - 1 (W - 1 when W <= G), is the last to touch the counter:
  // it tags the word with the next launch's epoch and hands the caller's
  // work_counter the value the reference's counter ends at (W + G, for the
  // report tile's queue length).  Drawn by lane 0 only, in two halves: the
  // atomic add is issued inside a tile's K loop and its value is looked at
  // only once the tile's K loop is done (a branch on it inside the loop would
  // make the wave wait for every DMA it has in flight).
  // (Not on the fp8 256x256 tile: it sits at the register limit, and the
  // bookkeeping made it spill more for no gain there.)
  constexpr bool kStaticRounds = MGG_STATIC_ROUNDS && !(T::kScaled && BM == 256 && BN == 256);
  // (dyn_base = S * G, recomputed where used: every value kept live through
  // the kernel costs registers the K loop needs.  Ticket-drawn tiles land on
  // whichever XCD is free first, so their A and B blocks are fetched by
  // several L2s; static rounds with partial m-tiles, whose costs differ,
  // measured faster all the same: expert-MLP forward -1.1 to -2.8%.)
  auto dyn_base = [&]() -> int32_t {
    if constexpr (kStaticRounds) {
      if (p.atomic && p.num_work < 0 && W_tiles >= 2 * G) return W_tiles / G * G;
    }
    return G;
  };
  // Whether the item after `item` is drawn by ticket (else it is item + G):
  // a worker's stripes are below dyn_base, drawn items at or above it.
  auto by_ticket_after = [&](int32_t item) -> bool {
    if constexpr (!kStaticRounds) return p.atomic != 0;
    return p.atomic && item + G >= dyn_base();
  };
  auto resolve = [&](unsigned long long raw) -> int32_t {
    const int32_t t = ticket_from(raw, p.counter, p.epoch);
    if constexpr (kStaticRounds) {
      if (t == (W > G ? W - dyn_base() + G - 1 : W - 1)) {
        __hip_atomic_store(p.counter, (unsigned long long)p.next_epoch << 32, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
        if (p.report != nullptr) atomicExch(p.report, w_report + G);
      }
      return dyn_base() + t;
    } else {
      if (t == W - 1) {
        __hip_atomic_store(p.counter, (unsigned long long)p.next_epoch << 32, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
        if (p.report != nullptr) atomicExch(p.report, w_report + G);
      }
      return G + t;
    }
  };
  auto draw = [&]() -> int32_t { return resolve(atomicAdd(p.counter, 1ull)); };
  // K < 2^30 (the host bounds (K+8)*ldb_k*2 below 2^31), so stage positions
  // are 32-bit and the full/partial decision stays in scalar registers.
  // K extent of the tile being issued (set by set_sources): all of K, or one
  // half of it for a split tile.
  int k_size = (int)K;
  int nk = (int)((K + kBK - 1) / kBK);

  const int64_t last_row = p.m - 1;

  // ---- tile decode ---------------------------------------------------------
  // The output tile of queue item `item`: expert e, rows [row_base,
  // row_base + rows_valid) of C, columns [n0, n0 + BN).  False for an item a
  // caller-built queue fills with an out-of-range or empty tile (skipped).
  struct Coords {
    int32_t e;
    int64_t row_base;
    int rows_valid;
    int64_t n0;
    int32_t slot;  // -1: the whole tile; s*t + q: part q of K of split tile t
  };
  auto decode = [&](int32_t item, Coords& c) -> bool {
    c.slot = -1;
    if (item >= w_base) {  // a part of a split tile
      c.slot = item - w_base;
      item = w_base + c.slot / split_s;
    }
    int e, tm, tn;
    if (p.num_work >= 0) {
      e = p.q_expert[item];
      tm = p.q_tile_m[item];
      tn = p.q_tile_n[item];
    } else {
      int lo = 0, hi = p.num_experts - 1;
      while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (s_prefix[mid] <= item) lo = mid; else hi = mid - 1;
      }
      e = lo;
      const int32_t local = item - s_prefix[e];
      // Within expert e: groups of MGG_GROUP_M m-tiles (the last group may
      // hold fewer, gm), each taken n-tile by n-tile, the group's m-tiles
      // consecutive.  The striped placement gives an XCD G/8 consecutive
      // items: with 32 n-tiles (N = 8192 at 256 columns) an XCD's 32 items
      // are 4 m-tiles x 8 n-tiles, 4 A blocks and 8 B blocks for its L2 to
      // share, against 1 A block and 32 B blocks in row order (the expert-MLP
      // up GEMM 2.2-4.6% faster); where the XCD's share already spans whole
      // m-tile rows (N = 4096 and 2048 here) it holds the same tiles as in
      // row order.
      if constexpr (MGG_GROUP_M > 1) {
        const int64_t cnt = (int64_t)(s_offs != nullptr ? s_offs[e + 1] : p.offsets[e + 1]) -
                            (s_offs != nullptr ? s_offs[e] : p.offsets[e]);
        const int32_t mt_e = (int32_t)((cnt + BM - 1) / BM);
        const int32_t span = MGG_GROUP_M * n_tiles;
        const int32_t g = local / span;
        const int32_t gm = min(MGG_GROUP_M, mt_e - g * MGG_GROUP_M);
        const int32_t sub = local - g * span;
        tn = sub / gm;
        tm = g * MGG_GROUP_M + (sub - tn * gm);
      } else {
        tm = local / n_tiles;
        tn = local - tm * n_tiles;
      }
    }
    // Uniform across the workgroup (memory reads look divergent to the
    // compiler): keep the coordinates, and all derived from them, in SGPRs.
    e = __builtin_amdgcn_readfirstlane(e);
    tm = __builtin_amdgcn_readfirstlane(tm);
    tn = __builtin_amdgcn_readfirstlane(tn);
    if ((uint32_t)e >= (uint32_t)p.num_experts || tm < 0 || (uint32_t)tn >= (uint32_t)n_tiles)
      return false;
    const int32_t off_lo = __builtin_amdgcn_readfirstlane(s_offs != nullptr ? s_offs[e] : p.offsets[e]);
    const int32_t off_hi =
        __builtin_amdgcn_readfirstlane(s_offs != nullptr ? s_offs[e + 1] : p.offsets[e + 1]);
    const int64_t m0 = (int64_t)tm * BM;
    const int64_t left = (int64_t)off_hi - off_lo - m0;
    if (left <= 0) return false;
    c.e = e;
    c.row_base = off_lo + m0;
    c.rows_valid = left < BM ? (int)left : BM;
    c.n0 = (int64_t)tn * BN;
    return true;
  };

  // ---- DMA sources ---------------------------------------------------------
  // Each descriptor ends exactly at the last element the tile may use, so a
  // DMA past it writes zeros and reads no memory: A's descriptor ends at the
  // tile's last valid row (rows past the expert's count, or past M, cost no
  // traffic; their results are never stored), B's at the last row of K.
  // K-major B is handled like A (rows of B past N read zeros).  N-major B
  // columns past N (edge tiles) are clamped onto the last 8 columns.  Offsets
  // are 32-bit (the host bounds lda and ldb_k).  ldb_k is the stride between
  // B's rows: K rows for N-major B, N rows for K-major B.
  auto a_swz = [](int r) {
    return kALdsChunks == 2 ? (r >> 3) & 1 : kALdsChunks == 4 ? (r >> 2) & 3 : (r >> 1) & 7;
  };
  // Chunk (row, K position) moved by lane `lane` in the t-th DMA of an A slot.
  auto a_row = [&](int t) { return kARowsPerDmaL * (wave * kAPerWave + t) + lane / kALdsChunks; };
  auto a_kpos = [&](int t) { return kChunkElems * ((lane % kALdsChunks) ^ a_swz(a_row(t))); };
  auto b_krow = [&](int t) { return (wave * kBPerWave + t) * kBRowsPerDma + lane / kBChunks; };
  // K-major B: row n of the tile and the K position of the chunk.
  auto b_kpos = [&](int t) { return kChunkElems * ((lane % kBChunks) ^ a_swz(b_krow(t))); };
  // Per-lane source offsets (bytes, stage 0): the same for every tile, or
  // with gathered A (A-block tile) per tile from the rows' indices.
  uint32_t a_voff[kAPerWave];
#pragma unroll
  for (int t = 0; t < kAPerWave; ++t) a_voff[t] = (uint32_t)((a_row(t) * p.lda + a_kpos(t)) * kE);
  // EPI: the epilogue (low two bits), plus kEpiGather for gathered A.
  constexpr int kEpi = EPI & 3;
  constexpr bool gathered = (EPI & kEpiGather) != 0;
  // The odd-N instance; with N-major 16-bit B it adds the term of B's last
  // element itself (odd_n_fix; SwiGLU's N is always even).
  constexpr bool kOddN = (EPI & kEpiOddN) != 0;
  constexpr bool kOddNFix = kOddN && !T::kBKMajor && !T::kScaled && kEpi != kEpiSwiglu;
  static_assert(!gathered || kABlk, "gathered A is built on the A-block tile");
  int32_t a_tok[kAPerWave];  // gathered A: source row of each of this lane's A rows, or -1
  const uint32_t b_row_bytes = (uint32_t)(p.ldb_k * kE);
  const uint32_t lds_a0 = lds_addr(lds);
  const uint32_t lds_b0 = lds_a0 + kASlots * kASlot;
  const uint8_t* a_bytes = reinterpret_cast<const uint8_t*>(p.a);
  const uint8_t* b_bytes = reinterpret_cast<const uint8_t*>(p.b);

  // The DMA state of the tile whose stages are being issued (and, for scaled
  // types, its coordinates and the LDS buffer its scales go to).
  i32x4 a_rsrc, b_rsrc;
  uint32_t b_voff[kBPerWave];
  Coords iss{};
  int iss_scale_buf = 0;
  // Scale buffer of the tile being multiplied: it alternates per tile, so the
  // next tile's scales can arrive while this tile's epilogue reads its own.
  int scale_buf = 0;
  auto set_sources = [&](const Coords& c, int scale_slot) {
    iss = c;
    iss_scale_buf = scale_slot;
    int64_t r0 = c.row_base;
    r0 = r0 < 0 ? 0 : (r0 > p.m ? p.m : r0);
    const int64_t r_end = c.row_base + c.rows_valid < p.m ? c.row_base + c.rows_valid : p.m;
    // A split part reads K [kb, ke): its descriptors start at kb and end at
    // ke, so every stage offset below is relative to kb.
    int kb = 0, klen = (int)K;
    if (c.slot >= 0) {
      const int q = c.slot % split_s;
      // Granule boundary before part pb (pb = 1 .. s-1): part q's share is
      // c - d * popcount(q) granules, c = (n_gran + d * P) / s, where d =
      // kSplitStagger and P sums popcount(q) over the s parts (see there).
      auto pc_sum = [](int pb) {  // popcount(0) + ... + popcount(pb - 1)
        int t = 0;
        for (int j = 1; j < pb; ++j) t += __builtin_popcount(j);
        return t;
      };
      auto bound = [&](int pb) {
        return pb * (n_gran + kSplitStagger * pc_sum(split_s)) / split_s - kSplitStagger * pc_sum(pb);
      };
      kb = q == 0 ? 0 : bound(q) * kGran;
      const int ke = q == split_s - 1 ? (int)K : bound(q + 1) * kGran;
      klen = ke - kb;
    }
    k_size = klen;
    nk = (klen + kBK - 1) / kBK;
    // A's rows are read to the next multiple of 8 columns past the item's K
    // range: with K not a multiple of 8, the 16-byte chunk that holds K-1
    // also holds columns up to that multiple (they meet B rows past K, which
    // read as zeros).
    const int64_t klen_a = (klen + 7) & ~7;
    if constexpr (gathered) {  // rows anywhere in the source matrix; per-lane offsets from set_a_rows
      const int64_t a_end = p.a_src_rows > 0 ? ((p.a_src_rows - 1) * p.lda + klen_a) * kE : 0;
      a_rsrc = make_rsrc4(a_bytes + (int64_t)kb * kE, a_end);
    } else {
      const int64_t a_end = r0 < r_end ? ((r_end - 1 - r0) * p.lda + klen_a) * kE : 0;
      a_rsrc = make_rsrc4(a_bytes + (r0 * p.lda + kb) * kE, a_end);
    }
    if constexpr (T::kBKMajor) {
      const int64_t b_end = c.n0 < p.n ? ((p.n - 1 - c.n0) * p.ldb_k + klen) * kE : 0;
      b_rsrc = make_rsrc4(b_bytes + ((int64_t)c.e * p.ldb_e + c.n0 * p.ldb_k + kb) * kE, b_end);
#pragma unroll
      for (int t = 0; t < kBPerWave; ++t)
        b_voff[t] = (uint32_t)((b_krow(t) * p.ldb_k + b_kpos(t)) * kE);
    } else {
      // N odd: the range check passes or zeroes whole dwords, and the dword
      // that holds a row's last element (N-1, even, so it starts the dword)
      // also holds the element after it.  The descriptor covers that element
      // when it lies inside B's view (a next row of this expert, or a next
      // expert); otherwise (the view's last element) B[e][K-1][N-1] reads as
      // zero and odd_n_fix adds its term.
      const bool tail_word =
          kOddN && (p.n & 1) && (kb + klen < K || (p.ldb_e > 0 && c.e < p.num_experts - 1));
      const int64_t b_end = ((klen - 1) * p.ldb_k + p.n - c.n0) * 2 + (tail_word ? 2 : 0);
      b_rsrc = make_rsrc4(b_bytes + ((int64_t)c.e * p.ldb_e + c.n0 + kb * p.ldb_k) * 2, b_end);
#pragma unroll
      for (int t = 0; t < kBPerWave; ++t) {
        const int k = b_krow(t);
        const int swz = BN >= 128 ? 4 * (k & 3) : 4 * ((k >> 1) & 1);
        const int64_t col = 8 * ((lane % kBChunks) ^ swz);
        // A chunk wholly past N reads the row's last 8 columns instead
        // (its outputs are never stored; N < 8: zeros); the chunk that holds
        // column N-1 (N not a multiple of 8) is read as it lies, its columns
        // past N coming from the next row, or as zeros past the descriptor.
        if (c.n0 + col < p.n)
          b_voff[t] = (uint32_t)((k * p.ldb_k + col) * 2);
        else
          b_voff[t] = p.n >= 8 ? (uint32_t)((k * p.ldb_k + p.n - 8 - c.n0) * 2) : kOutOfRange;
      }
    }
  };

  // Gathered A: load the source row index of each of this lane's A rows of
  // tile c (ordinary loads, issued ahead of their use), then turn them into
  // the lane's DMA offsets.  Rows past the tile's valid rows, and indices
  // outside the source matrix, get offsets past the descriptor (zeros).
  // Only entries inside [0, M) of the index array are read: a tile whose
  // rows fall outside it (offsets past M or negative) gets zero rows.
  auto load_rows = [&](const Coords& c) {
#pragma unroll
    for (int t = 0; t < kAPerWave; ++t) {
      const int64_t r = c.row_base + a_row(t);
      a_tok[t] = a_row(t) < c.rows_valid && r >= 0 && r < p.m ? p.a_rows[r] : -1;
    }
  };
  auto set_a_rows = [&]() {
#pragma unroll
    for (int t = 0; t < kAPerWave; ++t)
      a_voff[t] = a_tok[t] >= 0 && a_tok[t] < p.a_src_rows
                      ? (uint32_t)(((int64_t)a_tok[t] * p.lda + a_kpos(t)) * kE)
                      : kOutOfRange;
  };

  // Issues DMAs [d0, d1) of this wave's kDmaPerStage DMAs of stage s (the
  // first kAPerWave move A, the rest B) into LDS buffer s % kStages.  A full
  // stage keeps the stage offset in the SGPR offset; the partial last stage
  // puts it in the VGPR offset and redirects chunks at k >= K past the
  // descriptor, which makes the DMA write zeros.
  // The 128x512 tile serves experts of at most 128 rows (one m-tile each), so
  // its B lines are read by one tile only: they go with the non-temporal hint
  // and leave L2 to the A lines the expert's other n-tiles read (the
  // reference benchmark's problem: -2.1% striped, -2.9% atomic).
  constexpr bool kBStream = MGG_BSTREAM && BN == 512 && !T::kBKMajor;
  // FULL (a compile-time flag): the caller knows stage s lies wholly inside
  // K, so no DMA of it needs the partial-stage path.
  // buf: the LDS buffer of stage s (s % kStages), a constant where the
  // caller knows it.
  auto issue_part_f = [&](auto FULL, int s, int d0, int d1, int buf) {
    const int k0 = s * kBK;
    const uint32_t la = lds_a0 + buf * kAStage + wave * kAPerWave * 1024;
    const uint32_t lb = lds_b0 + buf * kBStage + wave * kBPerWave * 1024;
    const bool full = decltype(FULL)::value != 0 || k0 + kBK <= k_size;
#pragma unroll
    for (int d = d0; d < d1; ++d) {
      if (d < kAPerWave) {
        const int t = d;
        if (full) {
          dma16(a_rsrc, a_voff[t], (uint32_t)k0 * kE, la + t * 1024);
        } else {
          const uint32_t v = k0 + a_kpos(t) < k_size ? a_voff[t] + (uint32_t)k0 * kE : kOutOfRange;
          dma16(a_rsrc, v, 0u, la + t * 1024);
        }
      } else {
        const int t = d - kAPerWave;
        if constexpr (T::kBKMajor) {
          if (full) {
            dma16(b_rsrc, b_voff[t], (uint32_t)k0 * kE, lb + t * 1024);
          } else {
            const uint32_t v =
                k0 + b_kpos(t) < k_size ? b_voff[t] + (uint32_t)k0 * kE : kOutOfRange;
            dma16(b_rsrc, v, 0u, lb + t * 1024);
          }
        } else if (full) {
          if constexpr (kBStream)
            dma16_nt(b_rsrc, b_voff[t], (uint32_t)k0 * b_row_bytes, lb + t * 1024);
          else
            dma16(b_rsrc, b_voff[t], (uint32_t)k0 * b_row_bytes, lb + t * 1024);
        } else {
          const uint32_t v =
              k0 + b_krow(t) < k_size ? b_voff[t] + (uint32_t)k0 * b_row_bytes : kOutOfRange;
          dma16(b_rsrc, v, 0u, lb + t * 1024);
        }
      }
    }
  };
  auto issue_part = [&](int s, int d0, int d1) { issue_part_f(IntConst<0>{}, s, d0, d1, s % kStages); };
  // Scaled types: the tile's BM row scales and BN column scales go to its LDS
  // scale buffer by DMA with its stage 0 (one 64-word DMA per wave for the
  // first (BM+BN)/64 waves), so the first stage wait covers them; rows past
  // the tile's valid rows and columns past N read as zeros (descriptor ends).
  auto issue_scales = [&]() {
    if constexpr (T::kScaled) {
      static_assert(BM % 64 == 0 && BN % 64 == 0 && (BM + BN) / 64 <= NW, "one scale DMA per wave");
      if ((int)wave < (BM + BN) / 64) {
        const uint32_t dst = lds_addr(s_scale + iss_scale_buf * (BM + BN) + 64 * wave);
        // The lane offsets come from an opaque copy of the lane index: kept
        // live from the kernel's start they were spilled, and their reload
        // waited for every DMA in flight (vmcnt(0)) once per tile.
        int ol = lane;
        asm volatile("" : "+v"(ol));
        if (64 * (int)wave < BM) {
          int64_t rows = p.m - iss.row_base;
          rows = rows < iss.rows_valid ? rows : iss.rows_valid;
          const i32x4 rs = make_rsrc4(p.a_scale + (iss.row_base > 0 ? iss.row_base : 0),
                                      iss.row_base >= 0 && rows > 0 ? rows * 4 : 0);
          dma4(rs, (uint32_t)(64 * wave + ol) * 4, dst);
        } else {
          int64_t cols = p.n - iss.n0;
          cols = cols < BN ? cols : BN;
          const i32x4 rs = make_rsrc4(p.b_scale + (int64_t)iss.e * p.n + iss.n0, cols > 0 ? cols * 4 : 0);
          dma4(rs, (uint32_t)(64 * wave - BM + ol) * 4, dst);
        }
      }
    }
  };
  auto issue_stage = [&](int s) {
    issue_part(s, 0, kDmaPerStage);
    if (s == 0) issue_scales();
  };

  // ---- fragment addresses (LDS bytes, stage 0) ----------------------------
  const int frag_row = lane & 31;
  const int half = lane >> 5;
  // A fragment of K step kk: chunks kk*kStepChunks + half*kFragChunks + q of
  // row frag_row (+32j rows per block, the same swizzle).
  const uint32_t a_frag0 = (uint32_t)((wm * (BM / 2) + frag_row) * kALdsRow);
  // [half of an A block (kABlk; else 0)][K step][chunk]
  uint32_t a_off[kABlk ? 2 : 1][kSteps][kFragChunks];
#pragma unroll
  for (int h = 0; h < (kABlk ? 2 : 1); ++h)
#pragma unroll
    for (int kk = 0; kk < kSteps; ++kk)
#pragma unroll
      for (int q = 0; q < kFragChunks; ++q)
        a_off[h][kk][q] =
            lds_a0 + a_frag0 +
            (uint32_t)((((h * kSteps + kk) * kStepChunks + half * kFragChunks + q) ^ a_swz(frag_row)) * 16);
  const int tg = lane >> 4, ts = lane & 15;  // transposing-read group and source lane
  const int b_row_l = 8 * (tg >> 1) + (ts >> 2);
  const int b_swz = BN >= 128 ? 4 * ((ts >> 2) & 3) : 4 * ((ts >> 3) & 1);
  uint32_t b_off[kNB];  // N-major B: transposing-read address of block i (stage 0, K step 0)
  uint32_t bk_off[kSteps][kFragChunks];  // K-major B: like A, rows wn*(BN/kWN) + frag_row
#pragma unroll
  for (int i = 0; i < kNB; ++i) {
    const int n = wn * (BN / kWN) + 32 * i + 16 * (tg & 1) + 4 * (ts & 3);
    b_off[i] = lds_b0 + (uint32_t)(b_row_l * kBRowBytes + (((n >> 3) ^ b_swz) * 16) + (n & 7) * 2);
  }
  const int b_frag_row = wn * (BN / kWN) + frag_row;
#pragma unroll
  for (int kk = 0; kk < kSteps; ++kk)
#pragma unroll
    for (int q = 0; q < kFragChunks; ++q)
      bk_off[kk][q] = lds_b0 + (uint32_t)(b_frag_row * kBRowBytes) +
                      (uint32_t)(((kk * kStepChunks + half * kFragChunks + q) ^ a_swz(b_frag_row)) * 16);

  f32x16 acc[kNB][kMB];
  // Fragments are double-buffered by the parity of the K step's global index
  // (k0/16): buffer f holds the step being multiplied while the other fills.
  // kASingle (the fp8 256x256 tile, whose double-buffered 32-byte fragments
  // do not fit beside its accumulators): one A buffer; the MFMAs go by A
  // block, and each block's fragment of the next K step is read as soon as
  // that block's MFMAs have issued, a K step before it is needed.
  constexpr bool kASingle = T::kScaled && BM == 256 && BN == 256 && !kABlk && kMB == 4;
  using Frag = typename T::Frag;
  Frag fa[kASingle ? 1 : 2][kMB];
  Frag fb[2][kNB];
  // One fragment from kFragChunks 16-byte LDS reads at byte offsets off[q] + delta.
  auto read_rows = [&](const uint32_t* off, uint32_t delta) {
    Frag v;
#pragma unroll
    for (int q = 0; q < kFragChunks; ++q) {
      const u32x4 w = lds_load(lds, off[q] + delta - lds_a0);
#pragma unroll
      for (int x = 0; x < 4; ++x) v[4 * q + x] = w[x];
    }
    return v;
  };
  auto read_a = [&](int f, int buf, int kk, int j) {
    fa[kASingle ? 0 : f][j] = read_rows(a_off[0][kk], buf * kASlot + 32 * kALdsRow * j);
  };
  auto read_b = [&](int f, int buf, int kk, int i) {
    if constexpr (T::kBKMajor) {
      fb[f][i] = read_rows(bk_off[kk], buf * kBStage + 32 * kBRowBytes * i);
      return;
    }
    const uint32_t base = b_off[i] + buf * kBStage + 16 * kk * kBRowBytes - lds_a0;
    const i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (lds_i16x4*)(lds_ptr(lds) + base));
    const i16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (lds_i16x4*)(lds_ptr(lds) + base + 4 * kBRowBytes));
    const u32x2 l2 = __builtin_bit_cast(u32x2, lo);
    const u32x2 h2 = __builtin_bit_cast(u32x2, hi);
    Frag v;
    v[0] = l2[0];
    v[1] = l2[1];
    v[2] = h2[0];
    v[3] = h2[1];
    fb[f][i] = v;
  };
  // Half `part` of the fragments of K step kk of LDS buffer `buf`, into fragment buffer f.
  // with_a = 0: B only (kASingle reads A by block beside the MFMAs); 1: both;
  // -1: both unless kASingle.
  auto read_kstep = [&](int f, int buf, int kk, int part, int with_a = -1) {
    if (with_a == 1 || (with_a < 0 && !kASingle)) {
#pragma unroll
      for (int j = part * kMB / 2; j < (part + 1) * kMB / 2 + (kMB == 1 && part == 0); ++j)
        read_a(f, buf, kk, j);
    }
#pragma unroll
    for (int i = part * kNB / 2; i < (part + 1) * kNB / 2 + (kNB == 1 && part == 0); ++i)
      read_b(f, buf, kk, i);
  };
  auto mfma_group = [&](int f, int g) {  // quarter g of the MFMAs of fragment buffer f
    constexpr int kPer = kMB * kNB;
#pragma unroll
    for (int q = g * kPer / 4; q < (g + 1) * kPer / 4; ++q) {
      // kASingle: group g is A block g against every B block.
      const int i = kASingle ? q % kNB : q / kMB, j = kASingle ? q / kNB : q % kMB;
      acc[i][j] = T::mfma(fb[f][i], fa[kASingle ? 0 : f][j], acc[i][j]);
    }
  };

  // Waits until this wave's DMAs of every stage up to `s` are complete, given
  // that stages up to `last_issued` have been issued (each stage is
  // kDmaPerStage DMAs, and DMAs complete in issue order).
  auto wait_stage = [&](int s, int last_issued) {
    wait_dma_groups<kDmaPerStage, kStages - 2>(last_issued - s);
  };

  // MFMA groups of a stage in program order.  Each K step's 4 groups are
  // followed by: the next K step's fragment reads (half after group 0, half
  // after group 1, so they have two groups of MFMAs to land), and a share of
  // the DMAs of stage kt+kStages-1 (spread over the early groups so a wave
  // never stalls behind a burst of them; a one-step stage issues them all
  // first).  In the last K step the barrier that publishes stage kt+1 comes
  // after group 0 (by then every fragment of this stage has been read), and
  // stage kt+1's first fragments are read after groups 1 and 2.  P0 is the
  // fragment buffer of the stage's first K step, a compile-time constant.
  int issued = -1;
  constexpr int kEarlyGroups = kSteps > 1 ? 4 * (kSteps - 1) : 1;
  auto dma_share = [&](auto FULL, int grp, int s, int sbuf) {
    const int d0 = grp * kDmaPerStage / kEarlyGroups;
    const int d1 = (grp + 1) * kDmaPerStage / kEarlyGroups;
    if (d1 > d0) issue_part_f(FULL, s, d0, d1, sbuf);
  };
  auto early_steps = [&](auto P0, auto FULL, int buf, int next_stage, int next_buf, bool issue) {
    constexpr int p0 = decltype(P0)::value;
#pragma unroll
    for (int kk = 0; kk + 1 < kSteps; ++kk) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        mfma_group((p0 + kk) & 1, g);
        if constexpr (kASingle) read_a(0, buf, kk + 1, g);
        if (g < 2) read_kstep((p0 + kk + 1) & 1, buf, kk + 1, g);
        if (decltype(FULL)::value != 0 || issue) dma_share(FULL, kk * 4 + g, next_stage, next_buf);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
  };
  // A stage that has a successor to publish.  FULL: the stage it issues,
  // kt+kStages-1, lies wholly inside K (so it is issued, and its wait counts
  // kStages-2 stages issued after kt+1).  BUFC: kt % kStages when the caller
  // knows it at compile time (else -1), so LDS addresses fold to constants.
  auto stage = [&](auto P0, auto FULL, auto BUFC, int kt) {
    constexpr int p0 = decltype(P0)::value;
    constexpr bool full = decltype(FULL)::value != 0;
    constexpr int bc = decltype(BUFC)::value;
    constexpr int f_last = (p0 + kSteps - 1) & 1;
    constexpr int f_next = (p0 + kSteps) & 1;
    const int buf = bc >= 0 ? bc : kt % kStages;
    // Stage kt+kStages-1 goes into the buffer stage kt-1 used; every wave
    // finished reading it before the barrier of stage kt-1.
    const int ibuf = bc >= 0 ? (bc + kStages - 1) % kStages : (kt + kStages - 1) % kStages;
    const bool issue = full || kt + kStages - 1 < nk;
    if (issue) issued = kt + kStages - 1;
    if constexpr (kSteps == 1) {
      if (issue) issue_part_f(FULL, kt + kStages - 1, 0, kDmaPerStage, ibuf);
    }
    early_steps(P0, FULL, buf, kt + kStages - 1, ibuf, issue);
    mfma_group(f_last, 0);
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (full)
      wait_dma<(kStages - 2) * kDmaPerStage>();
    else
      wait_stage(kt + 1, issued);
    __syncthreads();
    const int nbuf = bc >= 0 ? (bc + 1) % kStages : (kt + 1) % kStages;
    if constexpr (kASingle) read_a(0, nbuf, 0, 0);
    mfma_group(f_last, 1);
    if constexpr (kASingle) read_a(0, nbuf, 0, 1);
    read_kstep(f_next, nbuf, 0, 0);
    __builtin_amdgcn_sched_barrier(0);
    mfma_group(f_last, 2);
    if constexpr (kASingle) read_a(0, nbuf, 0, 2);
    read_kstep(f_next, nbuf, 0, 1);
    __builtin_amdgcn_sched_barrier(0);
    mfma_group(f_last, 3);
    if constexpr (kASingle) read_a(0, nbuf, 0, 3);
    __builtin_amdgcn_sched_barrier(0);
  };
  auto last_stage = [&](auto P0, int kt) {
    constexpr int p0 = decltype(P0)::value;
    early_steps(P0, IntConst<0>{}, kt % kStages, 0, 0, false);
#pragma unroll
    for (int g = 0; g < 4; ++g) mfma_group((p0 + kSteps - 1) & 1, g);
  };
  // All stages of the current tile; stages 0 .. min(kStages-1, nk)-1 have
  // been issued (with a scaled type's scales, in LDS scale buffer scale_buf).
  // Returns after the last stage's fragments have been read and its MFMAs
  // issued.
  // ---- A in blocks of two stages (kABlk) -----------------------------------
  // Stage s multiplies A block s/2 (LDS slot (s/2)&1, K half s&1) and B stage s
  // (slot s % kBSlots).  Stage s issues, when s is even, A block s/2+1 (into
  // the slot block s/2-1 left; its four DMAs first), then B stage s+kLB (into
  // the slot stage s-1 left).  Loads past K are issued all the same (zeros,
  // no memory reads: offsets past the descriptors), so every wait counts a
  // fixed number of later DMAs: 4 after a stage of odd index (the A block of
  // the next stage is the last load it needs), 8 (kLB 3) or 10 (kLB >= 4)
  // after one of even index, (kLB-1) B stages' worth at a tile's start.
  constexpr int kWaitOdd = 2 * kBPerWave;
  // Even kt, kLB 3: the last load stage kt+1 needs is B stage kt+1 (issued in
  // stage kt-2 after that stage's A block); after it come stage kt-1's B and
  // stage kt's A block and B.  kLB >= 4: it is A block kt/2 (issued first in
  // stage kt-2); after it come stage kt-2's B, stage kt-1's B and stage kt's
  // A block and B.
  constexpr int kWaitEven = kLB == 3 ? kBPerWave + kAPerWave + kBPerWave
                                     : kBPerWave + kBPerWave + kAPerWave + kBPerWave;
  static_assert(!kABlk || (kAPerWave % 2 == 0 && kBPerWave % 2 == 0), "A-block DMA shares come in halves");
  // FULL (a compile-time flag): the caller knows the block or stage lies
  // wholly inside K, so no DMA of it needs the partial-stage path.
  // aslot / bslot: the LDS slot (m & 1, st % kBSlots), constants where the
  // caller knows them.
  auto issue_ablock_f = [&](auto FULL, int m, int t0, int t1, int aslot) {  // DMAs [t0, t1) of A block m
    const int k0 = m * 2 * kBK;
    const uint32_t la = lds_a0 + aslot * kASlot + wave * kAPerWave * 1024;
    const bool full = decltype(FULL)::value != 0 || k0 + 2 * kBK <= k_size;
#pragma unroll
    for (int t = t0; t < t1; ++t) {
      if (full) {
        dma16(a_rsrc, a_voff[t], (uint32_t)k0 * kE, la + t * 1024);
      } else {
        const uint32_t v = k0 + a_kpos(t) < k_size ? a_voff[t] + (uint32_t)k0 * kE : kOutOfRange;
        dma16(a_rsrc, v, 0u, la + t * 1024);
      }
    }
  };
  auto issue_bstage_f = [&](auto FULL, int st, int d0, int d1, int bslot) {  // DMAs [d0, d1) of B stage st
    const int k0 = st * kBK;
    const uint32_t lb = lds_b0 + bslot * kBStage + wave * kBPerWave * 1024;
    const bool full = decltype(FULL)::value != 0 || k0 + kBK <= k_size;
#pragma unroll
    for (int t = d0; t < d1; ++t) {
      if (full) {
        dma16(b_rsrc, b_voff[t], (uint32_t)k0 * b_row_bytes, lb + t * 1024);
      } else {
        const uint32_t v =
            k0 + b_krow(t) < k_size ? b_voff[t] + (uint32_t)k0 * b_row_bytes : kOutOfRange;
        dma16(b_rsrc, v, 0u, lb + t * 1024);
      }
    }
  };
  auto issue_ablock = [&](int m, int t0, int t1) { issue_ablock_f(IntConst<0>{}, m, t0, t1, m & 1); };
  auto issue_bstage = [&](int st, int d0, int d1) {
    issue_bstage_f(IntConst<0>{}, st, d0, d1, st % kBSlots);
  };
  // Half `part` of the fragments of K step kk of stage st (A half H of its
  // block); q: st % 4 when the caller knows it at compile time (else -1).
  auto read_kstep_ab = [&](auto H, int f, int st, int kk, int part, int q = -1) {
    constexpr int h = decltype(H)::value;
    const int aslot = q >= 0 ? (q >> 1) & 1 : (st >> 1) & 1;
    const int bslot = q >= 0 && kBSlots == 4 ? q : st % kBSlots;
#pragma unroll
    for (int j = part * kMB / 2; j < (part + 1) * kMB / 2; ++j)
      fa[f][j] = read_rows(a_off[kABlk ? h : 0][kk], aslot * kASlot + 32 * kALdsRow * j);
#pragma unroll
    for (int i = part * kNB / 2; i < (part + 1) * kNB / 2 + (kNB == 1 && part == 0); ++i)
      read_b(f, bslot, kk, i);
  };
  // Stage kt of A half H (kt % 2 == H), in run_worker's stage order: K step 0
  // on fragment buffer 0 while step 1's fragments are read and this stage's
  // DMAs go out, then step 1, the wait and barrier for stage kt+1, and its
  // first fragments.
  // Q: kt % 4 when the caller knows it at compile time (else -1), so the LDS
  // slots fold to constants.
  auto stage_ab = [&](auto H, auto FULL, auto Q, int kt) {
    constexpr int h = decltype(H)::value;
    constexpr int q = decltype(Q)::value;
    const int aslot_next = q >= 0 ? ((q >> 1) + 1) & 1 : (kt / 2 + 1) & 1;
    const int bslot_next = q >= 0 && kBSlots == 4 ? (q + kLB) % 4 : (kt + kLB) % kBSlots;
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      mfma_group(0, g);
      if (g < 2) read_kstep_ab(H, 1, kt, 1, g, q);
      if constexpr (h == 0) {
        if (g < 2) issue_ablock_f(FULL, kt / 2 + 1, g * kAPerWave / 2, (g + 1) * kAPerWave / 2, aslot_next);
        else issue_bstage_f(FULL, kt + kLB, (g - 2) * kBPerWave / 2, (g - 1) * kBPerWave / 2, bslot_next);
      } else {
        if (g == 0 || g == 2)
          issue_bstage_f(FULL, kt + kLB, g / 2 * kBPerWave / 2, (g / 2 + 1) * kBPerWave / 2, bslot_next);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    mfma_group(1, 0);
    __builtin_amdgcn_sched_barrier(0);
    wait_dma<h == 0 ? kWaitEven : kWaitOdd>();
    __syncthreads();
    mfma_group(1, 1);
    read_kstep_ab(IntConst<1 - h>{}, 0, kt + 1, 0, 0, q >= 0 ? (q + 1) % 4 : -1);
    __builtin_amdgcn_sched_barrier(0);
    mfma_group(1, 2);
    read_kstep_ab(IntConst<1 - h>{}, 0, kt + 1, 0, 1, q >= 0 ? (q + 1) % 4 : -1);
    __builtin_amdgcn_sched_barrier(0);
    mfma_group(1, 3);
    __builtin_amdgcn_sched_barrier(0);
  };
  // A tile's first loads: A block 0, then B stages 0 .. kLB-1.
  auto prologue_ab = [&](bool first_only) {
    issue_ablock(0, 0, kAPerWave);
    issue_bstage(0, 0, kBPerWave);
    if (!first_only)
      for (int st = 1; st < kLB; ++st) issue_bstage(st, 0, kBPerWave);
  };

  auto main_loop = [&](bool take_ticket, unsigned long long& ticket) {
#pragma unroll
    for (int i = 0; i < kNB; ++i)
#pragma unroll
      for (int j = 0; j < kMB; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;
    if constexpr (kABlk)
      wait_dma<(kLB - 1) * kBPerWave>();  // B stages 1 .. kLB-1 issued after stage 0's B
    else
      wait_stage(0, issued);
    __syncthreads();
    // The next tile's ticket, taken after the first wait so that this
    // wave's first DMA wait does not also wait for the atomic; its value is
    // resolved after the K loop.
    if (take_ticket && tid == 0) ticket = atomicAdd(p.counter, 1ull);
    if constexpr (kABlk) {
      read_kstep_ab(IntConst<0>{}, 0, 0, 0, 0);
      read_kstep_ab(IntConst<0>{}, 0, 0, 0, 1);
      const int nk2 = (nk + 1) & ~1;  // pairs of stages; an odd count ends on a zero stage
      // Pairs whose issued A block (kt/2 + 1) and B stages (kt + kLB, kt + kLB
      // + 1) lie wholly inside K run without the partial-stage checks.
      // (B stage kt + 1 + kLB is full iff (kt + kLB + 2) * kBK <= K; the A block
      // kt/2 + 1 iff (kt + 4) * kBK <= K.)  A DMA on the full path keeps its
      // stage offset in the unchecked SGPR offset, so this bound must hold.
      const int kt_full = k_size / kBK - kLB - 2;  // kt <= kt_full: every issued stage full
      int kt = 0;
      if constexpr (MGG_FULL_LOOP) {
        // Two pairs per iteration from kt = 0 (kt % 4 known: constant slots).
        for (; kt + 2 < nk2 && kt + 2 <= kt_full; kt += 4) {
          stage_ab(IntConst<0>{}, IntConst<1>{}, IntConst<0>{}, kt);
          stage_ab(IntConst<1>{}, IntConst<1>{}, IntConst<1>{}, kt + 1);
          stage_ab(IntConst<0>{}, IntConst<1>{}, IntConst<2>{}, kt + 2);
          stage_ab(IntConst<1>{}, IntConst<1>{}, IntConst<3>{}, kt + 3);
        }
        for (; kt < nk2 && kt <= kt_full; kt += 2) {
          stage_ab(IntConst<0>{}, IntConst<1>{}, IntConst<-1>{}, kt);
          stage_ab(IntConst<1>{}, IntConst<1>{}, IntConst<-1>{}, kt + 1);
        }
      }
      for (; kt < nk2; kt += 2) {
        stage_ab(IntConst<0>{}, IntConst<0>{}, IntConst<-1>{}, kt);
        stage_ab(IntConst<1>{}, IntConst<0>{}, IntConst<-1>{}, kt + 1);
      }
      return;
    }
    if (nk > 0) {
      read_kstep(0, 0, 0, 0, 1);
      read_kstep(0, 0, 0, 1, 1);
    }
    int kt = 0;
    // Stages whose issued stage kt+kStages-1 lies wholly inside K run without
    // the partial-stage checks: kt <= kt_full.  (A DMA on the full path keeps
    // its stage offset in the unchecked SGPR offset, so this bound must hold.)
    const int kt_full = k_size / kBK - kStages;
    if constexpr (kSteps % 2 == 0) {  // every stage starts on fragment buffer 0
      if constexpr (MGG_FULL_LOOP) {
        // Full stages unrolled by the ring length from kt = 0, so each
        // stage's LDS buffer is a compile-time constant.
        for (; kt + kStages < nk && kt + kStages - 1 <= kt_full; kt += kStages)
          static_for<kStages>([&](auto B) { stage(IntConst<0>{}, IntConst<1>{}, B, kt + decltype(B)::value); });
        for (; kt + 1 < nk && kt <= kt_full; ++kt) stage(IntConst<0>{}, IntConst<1>{}, IntConst<-1>{}, kt);
      }
      for (; kt + 1 < nk; ++kt) stage(IntConst<0>{}, IntConst<0>{}, IntConst<-1>{}, kt);
      if (nk > 0) last_stage(IntConst<0>{}, kt);
    } else {  // one-step stages alternate buffers: unrolled by two
      if constexpr (MGG_FULL_LOOP) {
        for (; kt + 2 < nk && kt + 1 <= kt_full; kt += 2) {
          stage(IntConst<0>{}, IntConst<1>{}, IntConst<-1>{}, kt);
          stage(IntConst<1>{}, IntConst<1>{}, IntConst<-1>{}, kt + 1);
        }
      }
      for (; kt + 2 < nk; kt += 2) {
        stage(IntConst<0>{}, IntConst<0>{}, IntConst<-1>{}, kt);
        stage(IntConst<1>{}, IntConst<0>{}, IntConst<-1>{}, kt + 1);
      }
      if (kt + 1 < nk) {
        stage(IntConst<0>{}, IntConst<0>{}, IntConst<-1>{}, kt);
        last_stage(IntConst<1>{}, kt + 1);
      } else if (nk > 0) {
        last_stage(IntConst<0>{}, kt);
      }
    }
  };

  // ---- epilogue: acc[i][j] register r holds D[n][m] of the 32x32 block with
  // n = 8*(r/4) + 4*(lane/32) + r%4, m = lane%32 (D = C^T).  With the SwiGLU
  // epilogue B's columns come interleaved in groups of 64 (32 gate columns,
  // then the 32 up columns of the same outputs), so a wave's 32-column blocks
  // 2i and 2i+1 are gate and up of the same 32 outputs and C has N/2 columns.
  static_assert(kEpi != kEpiSwiglu || kNB % 2 == 0, "SwiGLU needs pairs of 32-column blocks per wave");
  static_assert(kEpi == kEpiNone || !T::kScaled, "fused epilogues are for unscaled types");
  // Stores: a lane holds 4 consecutive columns of each 8-column group g; the
  // lanes l and l+32 of one row swap halves of groups (2p, 2p+1) with
  // v_permlane32_swap so that each lane stores 8 consecutive columns (16 bytes)
  // and a row segment of 32 contiguous bytes goes out per pair of lanes.
  // y0: this lane's 4 values of group 2p, y1: of group 2p+1.  Returns the 8
  // consecutive columns the lane stores: lanes 0-31 the first 8 of the 16,
  // lanes 32-63 the last 8.
  auto pack_pair = [&](const float* y0, const float* y1) -> u32x4 {
    const uint32_t a0 = T::pack(y0[0], y0[1]), a1 = T::pack(y0[2], y0[3]);
    const uint32_t b0 = T::pack(y1[0], y1[1]), b1 = T::pack(y1[2], y1[3]);
    const auto s0 = __builtin_amdgcn_permlane32_swap(a0, b0, false, false);
    const auto s1 = __builtin_amdgcn_permlane32_swap(a1, b1, false, false);
    return u32x4{(uint32_t)s0[0], (uint32_t)s1[0], (uint32_t)s0[1], (uint32_t)s1[1]};
  };
  // 8 consecutive outputs at crow + col, of which those before column
  // `cols` are stored: one 16-byte store, or (the last chunk of a row when
  // the row length is not a multiple of 8) one store per pair, and in the
  // odd-N instance a 2-byte store for a last column of its own.
  auto store_chunk = [&](uint16_t* crow, int64_t col, int64_t cols, const u32x4& v) {
    if (col + 8 <= cols) {
      __builtin_nontemporal_store(v, reinterpret_cast<u32x4*>(crow + col));
    } else if (col < cols) {
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        if (!kOddN || col + 2 * w + 1 < cols) {
          if (col + 2 * w < cols)
            __builtin_nontemporal_store(v[w], reinterpret_cast<uint32_t*>(crow + col) + w);
        } else if (col + 2 * w < cols) {
          __builtin_nontemporal_store((uint16_t)v[w], crow + col + 2 * w);
        }
      }
    }
  };
  auto store_pair = [&](uint16_t* crow, int64_t col, int64_t cols, bool row_ok,
                        const float* y0, const float* y1) {
    const u32x4 v = pack_pair(y0, y1);
    // col already includes 8*half
    if (row_ok) store_chunk(crow, col, cols, v);
  };
  // Stores through LDS: a wave's output columns of a row are one 64-, 128-
  // or 256-byte segment of C, but a store instruction straight from the MFMA
  // layout writes 32 rows x 32 bytes.  Each 32-row block instead goes to an
  // LDS region of the wave (row r, 16-byte chunk ch at ch ^ swz(r),
  // conflict-free both ways) and comes back as whole row segments, 4 rows of
  // 256 bytes, 8 of 128 or 16 of 64 per instruction (32 MiB bursts of such
  // stores measured 30% faster than 32-byte segments for 128 bytes; 64-byte
  // ones 19% faster).  The LDS region is free for the whole epilogue:
  // * A-block tile: a 4 KiB share of A slot 1.  No DMA is in flight into it
  //   (the last stage's wait retired the zero-fill block the last even stage
  //   sent there) and the next tile first fills it in its first stage, after
  //   the barrier that opens its K loop.
  // * Other tiles: the wave's own share of buffer 1's A stage, or for
  //   256-byte rows (16 rows in each) its shares of buffers 1 and 2's B
  //   stages.  Every DMA has retired before the last stage (its wait is for
  //   all of them), and only this wave writes those shares: buffer 1 with the
  //   next tile's stage 1, issued after this wave's epilogue, buffer 2 with
  //   stage 2, issued after the next tile's first barrier.
  // The LDS addresses are derived from an opaque copy of the lane index taken
  // in the epilogue: otherwise the compiler computes them once per kernel and
  // keeps them live through the K loop, which then spills.
  // C goes out with non-temporal stores: this launch never reads it again, and
  // left in L2 it would evict A and B lines that other tiles still read
  // (measured: skewed routing and the atomic schedule 4-5.5% faster, fp8
  // 3.5-5%).
  constexpr int kOutCols = kEpi == kEpiSwiglu ? BN / kWN / 2 : BN / kWN;  // per wave and row
  constexpr int kLineChunks = kOutCols * 2 / 16;  // 16-byte chunks of a wave's row segment
  // 256-byte rows: the wave's shares of B stages 1 (rows 0-15) and 2 (16-31).
  constexpr bool kLine256 = kLineChunks == 16 && !kABlk && kStages >= 3 && kBPerWave * 1024 >= 16 * 256;
  constexpr bool kLineStores =
      kLine256 || ((kLineChunks == 4 || kLineChunks == 8) &&
                   (kABlk ? NW * 4096 <= kASlot : kStages >= 2 && kAPerWave * 1024 >= 32 * 16 * kLineChunks));
  const uint32_t line_region =
      kLine256 ? (uint32_t)(kASlots * kASlot + kBStage) + wave * (uint32_t)kBPerWave * 1024u
      : kABlk  ? (uint32_t)kASlot + wave * 4096u
               : (uint32_t)kAStage + wave * (uint32_t)kAPerWave * 1024u;
  auto opaque_lane = [&]() {
    int l = lane;
    asm volatile("" : "+v"(l));
    return l;
  };
  auto line_addr = [&](int r, int ch) {
    if constexpr (kLine256)
      return line_region + (uint32_t)((r >> 4) * kBStage + (r & 15) * 256 + ((ch ^ (r & 15)) * 16));
    const int swz = kLineChunks == 8 ? (r >> 1) & 7 : (r >> 2) & 3;
    return line_region + (uint32_t)(r * 16 * kLineChunks + ((ch ^ swz) * 16));
  };
  auto line_put = [&](int r, int ch, const u32x4& v) {
    *reinterpret_cast<__attribute__((address_space(3))) u32x4*>(lds_ptr(lds) + line_addr(r, ch)) = v;
  };
  // Row block j (32 rows) of this wave, all in LDS: store its row segments.
  // col0: C column of the wave's first output column; cols: C's columns.
  auto line_flush = [&](const Coords& c, int j, int ol, int64_t col0, int64_t cols) {
    // Lanes read what other lanes wrote: keep the compiler from moving LDS
    // accesses across this point (the hardware runs a wave's LDS operations
    // in order), here and after the reads.
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    __builtin_amdgcn_wave_barrier();
    constexpr int kRowsPer = 64 / kLineChunks;  // rows per store instruction
    const int ch = ol % kLineChunks;
    const int64_t col = col0 + 8 * ch;
#pragma unroll
    for (int q = 0; q < 32 / kRowsPer; ++q) {
      const int rr = kRowsPer * q + ol / kLineChunks;
      const u32x4 v =
          *reinterpret_cast<const __attribute__((address_space(3))) u32x4*>(lds_ptr(lds) + line_addr(rr, ch));
      const int mr = wm * (BM / 2) + 32 * j + rr;
      const int64_t gr = c.row_base + mr;
      if (mr < c.rows_valid && gr >= 0 && gr <= last_row) store_chunk(p.c + gr * p.ldc, col, cols, v);
    }
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    __builtin_amdgcn_wave_barrier();
  };
  auto epilogue = [&](const Coords& c) {
    const float* sc = s_scale + scale_buf * (BM + BN);
#pragma unroll
    for (int j = 0; j < kMB; ++j) {
      const int m = wm * (BM / 2) + 32 * j + frag_row;
      const float row_scale = T::kScaled ? sc[m] : 1.0f;
      const int64_t grow = c.row_base + m;
      const bool row_ok = m < c.rows_valid && grow >= 0 && grow <= last_row;
      uint16_t* crow = p.c + grow * p.ldc;
      const int ol = kLineStores ? opaque_lane() : lane;
      if constexpr (kEpi == kEpiSwiglu) {
#pragma unroll
        for (int ip = 0; ip < kNB / 2; ++ip) {
          const int64_t f0 = (c.n0 + wn * (BN / kWN) + 64 * ip) / 2;
#pragma unroll
          for (int pp = 0; pp < 2; ++pp) {
            float y0[4], y1[4];
#pragma unroll
            for (int q = 0; q < 4; ++q) {
              y0[q] = silu_mul(acc[2 * ip][j][8 * pp + q], acc[2 * ip + 1][j][8 * pp + q]);
              y1[q] = silu_mul(acc[2 * ip][j][8 * pp + 4 + q], acc[2 * ip + 1][j][8 * pp + 4 + q]);
            }
            if constexpr (kLineStores)
              line_put(ol & 31, 4 * ip + 2 * pp + (ol >> 5), pack_pair(y0, y1));
            else
              store_pair(crow, f0 + 16 * pp + 8 * half, p.n / 2, row_ok, y0, y1);
          }
        }
        if constexpr (kLineStores) line_flush(c, j, ol, (c.n0 + wn * (BN / kWN)) / 2, p.n / 2);
      } else {
#pragma unroll
        for (int i = 0; i < kNB; ++i) {
          const int cb = wn * (BN / kWN) + 32 * i;  // tile column of the block
#pragma unroll
          for (int pp = 0; pp < 2; ++pp) {
            float y[2][4];
#pragma unroll
            for (int h = 0; h < 2; ++h)
#pragma unroll
              for (int q = 0; q < 4; ++q) {
                const int g = 2 * pp + h;
                float v = acc[i][j][4 * g + q];
                if constexpr (T::kScaled) v *= row_scale * sc[BM + cb + 8 * g + 4 * half + q];
                y[h][q] = kEpi == kEpiGelu ? gelu_erf(v) : v;
              }
            if constexpr (kLineStores)
              line_put(ol & 31, 4 * i + 2 * pp + (ol >> 5), pack_pair(y[0], y[1]));
            else
              store_pair(crow, c.n0 + cb + 16 * pp + 8 * half, p.n, row_ok, y[0], y[1]);
          }
        }
        if constexpr (kLineStores) line_flush(c, j, ol, c.n0 + wn * (BN / kWN), p.n);
      }
    }
  };

  // N odd, 16-bit N-major B: where the element after B's last element
  // B[e][K-1][N-1] lies past B's view (the last expert, or every expert when
  // they share one B through ldb_e == 0), the K loop read that element as
  // zero (see set_sources).  Its term A[r][K-1] * B[e][K-1][N-1] is added to
  // the fp32 sums of column N-1 here, once per tile (after a split tile's
  // parts have met), by the lanes that hold that column.
  auto odd_n_fix = [&](const Coords& c) {
    if constexpr (kOddNFix) {
      const int64_t tc = p.n - 1 - c.n0;  // tile column of C's last column
      if (wn != (int)(tc / (BN / kWN))) return;
      const int cw = (int)(tc % (BN / kWN));
      // (lane values from an opaque copy of the lane index, so that nothing
      // derived here is kept live through the K loop)
      const int ol = opaque_lane();
      if ((ol >> 5) != (cw % 8) / 4) return;
      const int i_t = cw / 32, r_t = 4 * ((cw % 32) / 8) + cw % 4;
      const uint16_t* a16 = reinterpret_cast<const uint16_t*>(p.a);
      const uint16_t* b16 = reinterpret_cast<const uint16_t*>(p.b);
      const float bv = T::to_float(b16[(int64_t)c.e * p.ldb_e + (K - 1) * p.ldb_k + p.n - 1]);
#pragma unroll
      for (int j = 0; j < kMB; ++j) {
        const int m = wm * (BM / 2) + 32 * j + (ol & 31);
        const int64_t grow = c.row_base + m;
        if (m >= c.rows_valid || grow < 0 || grow > last_row) continue;
        int64_t ar = grow;
        if constexpr (gathered) {
          ar = p.a_rows[grow];
          if (ar < 0 || ar >= p.a_src_rows) continue;
        }
        const float t = T::to_float(a16[ar * p.lda + K - 1]) * bv;
#pragma unroll
        for (int i = 0; i < kNB; ++i)
#pragma unroll
          for (int r = 0; r < 16; ++r)
            if (i == i_t && r == r_t) acc[i][j][r] += t;
      }
    }
  };

  // ---- split tiles: the parts meet -------------------------------------------
  // A slot holds one part's (or a subtree's) partial sums: wave w's
  // accumulators as quads of 4 floats, quad g at byte (g * NW + w) * 1024 +
  // 16 * lane, so each store or load of a wave covers 1 KiB.  They go through
  // uncached memory with sc0 sc1 (no cache level holds a copy another XCD
  // could read stale).
  constexpr int kQuads = kNB * kMB * 4;
  auto partial_rsrc = [&](int32_t slot) {
    return __builtin_amdgcn_make_buffer_rsrc(p.split_partials + (int64_t)slot * BM * BN, (short)0,
                                             BM * BN * 4, 0x00020000);
  };
  auto write_partial = [&](int32_t slot) {
    const auto r = partial_rsrc(slot);
#pragma unroll
    for (int i = 0; i < kNB; ++i)
#pragma unroll
      for (int j = 0; j < kMB; ++j)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int g = (i * kMB + j) * 4 + q;
          // (Elements go through scalars: hipcc miscompiles __builtin_bit_cast
          // of a vector element, reading element 0 whatever the index.)
          const u32x4 v = {__float_as_uint(acc[i][j][4 * q]), __float_as_uint(acc[i][j][4 * q + 1]),
                           __float_as_uint(acc[i][j][4 * q + 2]), __float_as_uint(acc[i][j][4 * q + 3])};
          __builtin_amdgcn_raw_buffer_store_b128(v, r, (int)(wave * 1024 + 16 * lane), g * NW * 1024, 17);
        }
  };
  // Two 32x32 blocks (8 quads, 32 registers) in flight at a time: the
  // accumulators leave no room for more.
  auto add_partial = [&](int32_t slot) {
    const auto r = partial_rsrc(slot);
#pragma unroll
    for (int b0 = 0; b0 < kNB * kMB; b0 += 2) {
      u32x4 v[2][4];
#pragma unroll
      for (int bb = 0; bb < 2 && b0 + bb < kNB * kMB; ++bb)
#pragma unroll
        for (int q = 0; q < 4; ++q)
          v[bb][q] = __builtin_amdgcn_raw_buffer_load_b128(r, (int)(wave * 1024 + 16 * lane),
                                                           ((b0 + bb) * 4 + q) * NW * 1024, 17);
#pragma unroll
      for (int bb = 0; bb < 2 && b0 + bb < kNB * kMB; ++bb) {
        const int i = (b0 + bb) / kMB, j = (b0 + bb) % kMB;
#pragma unroll
        for (int q = 0; q < 4; ++q)
#pragma unroll
          for (int x = 0; x < 4; ++x) {
            const uint32_t u = v[bb][q][x];
            acc[i][j][4 * q + x] += __uint_as_float(u);
          }
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  static_assert(kQuads * 1024 * NW == BM * BN * 4, "a partial slot is the tile's fp32 sums");
  // The s parts of a split tile meet in a binary tree of s - 1 meetings.  At
  // level l a worker holds the sum of the parts [b, min(b + 2^l, s)) with
  // b = q & -2^l (its accumulators); when the sibling subtree, from
  // b ^ 2^l, exists (b ^ 2^l < s), the two holders meet on the level's flag
  // word for the pair, else the worker goes on to the next level alone.  At
  // a meeting a worker either finds the sibling finished (the flag reads
  // count 1 in this launch's epoch) or writes its sums to slot s*t + b,
  // waits until they are complete, and takes a ticket on the flag (the
  // dequeue's epoch-tagged claim, so a flag left by an unfinished launch
  // reads as fresh).  The worker that finds the sibling finished, or draws
  // ticket 1, returns the flag to 0, adds the sibling's sums from slot s*t +
  // (b ^ 2^l) and goes on to the next level; the other is done.  The worker
  // that completes the last level stores the tile (returns true).  fp32
  // addition is commutative, so every meeting's sum, and the tile, is the
  // same whichever worker arrives first, and no worker ever waits for
  // another.  Tile t's s - 1 flag words start at (s - 1) * t: level l's
  // pairs follow those of the levels below it, pair q >> (l + 1) of the
  // ceil(s / 2^l) subtrees at that level.
  auto split_fixup = [&](const Coords& c) -> bool {
    const int s = split_s;
    const int32_t t = c.slot / s;
    const int q = c.slot - t * s;
    int64_t level_flags = (int64_t)(s - 1) * t;  // first flag word of level l
    int subtrees = s;                              // ceil(s / 2^l)
    for (int l = 0; (1 << l) < s; ++l) {
      const int32_t b = q & -(1 << l);
      unsigned long long* flag = p.split_flags + level_flags + (q >> (l + 1));
      level_flags += subtrees >> 1;
      subtrees = (subtrees + 1) >> 1;
      if ((b ^ (1 << l)) >= s) continue;  // no sibling subtree at this level
      if (tid == 0) {
        const unsigned long long f = __hip_atomic_load(flag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        s_item[1] = ((uint32_t)(f >> 32) == p.epoch && (uint32_t)f == 1u) ? 1 : 0;
      }
      __syncthreads();
      bool last = s_item[1] != 0;
      __syncthreads();
      if (!last) {
        write_partial(s * t + b);
        wait_dma<0>();  // this wave's partial stores are complete (vmcnt counts stores too)
        __syncthreads();
        if (tid == 0) s_item[1] = first_ticket(flag, p.epoch) == 1 ? 1 : 0;
        __syncthreads();
        last = s_item[1] != 0;
        __syncthreads();
      }
      if (!last) return false;
      if (tid == 0) __hip_atomic_store(flag, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      add_partial(s * t + (b ^ (1 << l)));
    }
    return true;
  };

  // ---- the persistent loop -------------------------------------------------
  // Blocking ticket (used for the first item and to skip a caller queue's
  // invalid items): the leader takes it and broadcasts it through LDS.
  auto take_ticket_now = [&]() -> int32_t {
    if (tid == 0) *s_item = draw();
    __syncthreads();
    const int32_t t = *s_item;
    __syncthreads();
    return t;
  };
  auto advance = [&](int32_t item) -> int32_t {
    if constexpr (!kStaticRounds) return p.atomic ? take_ticket_now() : item + G;
    return by_ticket_after(item) ? take_ticket_now() : item + G;
  };
  // The first valid item at or after `item` (W or more when none is left).
  auto find_valid = [&](int32_t item, Coords& c) -> int32_t {
    while ((uint32_t)item < (uint32_t)W && !decode(item, c)) item = advance(item);
    return item;
  };

  Coords cur;
  int32_t w = find_valid(first, cur);
  if ((uint32_t)w >= (uint32_t)W) return;
  set_sources(cur, scale_buf);
  if constexpr (kABlk) {
    if constexpr (gathered) {
      load_rows(cur);
      set_a_rows();
    }
    prologue_ab(false);
  } else {
#pragma unroll
    for (int s = 0; s < kStages - 1; ++s)
      if (s < nk) issue_stage(issued = s);
  }
  for (;;) {
    unsigned long long ticket = 0;
    main_loop(kStaticRounds ? by_ticket_after(w) : p.atomic != 0, ticket);
    // The next item: the ticket taken during this tile, or the next stripe.
    // (Recomputed rather than kept live across the K loop.)
    if ((kStaticRounds ? by_ticket_after(w) : p.atomic != 0) && tid == 0) *s_item = resolve(ticket);
    __syncthreads();  // every wave is done reading this tile's LDS stages; s_item is visible
    int32_t next = (kStaticRounds ? by_ticket_after(w) : p.atomic != 0) ? *s_item : w + G;
    // A split part meets the others before anything of the next item is
    // issued (fewer registers live across the meetings).
    const bool store_cur = cur.slot < 0 || split_fixup(cur);
    if constexpr (kOddNFix)
      if (store_cur && (p.n & 1) && K > 0 && (p.ldb_e == 0 || cur.e == p.num_experts - 1) &&
          cur.n0 + BN >= p.n)
        odd_n_fix(cur);
    Coords nxt;
    next = find_valid(next, nxt);
    const bool more = (uint32_t)next < (uint32_t)W;
    // The next tile's first stage goes out before this tile's stores and its
    // other prologue stages after them, so each later wait only ever counts
    // DMAs issued after the stage it waits for.  Gathered A: the next tile's
    // row indices are loaded first and its B stage 0 goes out, the stores
    // cover the indices' latency, then A block 0 follows (the first wait
    // still finds B stages 1 .. kLB-1 issued after both).
    issued = -1;
    if (more) {
      set_sources(nxt, scale_buf ^ 1);
      if constexpr (kABlk) {
        if constexpr (gathered) {
          load_rows(nxt);
          issue_bstage(0, 0, kBPerWave);
        } else {
          prologue_ab(true);
        }
      } else if (nk > 0) {
        issue_stage(issued = 0);
      }
    }
    if (store_cur) epilogue(cur);
    if (!more) break;
    if constexpr (kABlk) {
      if constexpr (gathered) {
        set_a_rows();
        issue_ablock(0, 0, kAPerWave);
      }
      for (int st = 1; st < kLB; ++st) issue_bstage(st, 0, kBPerWave);
    } else {
#pragma unroll
      for (int s = 1; s < kStages - 1; ++s)
        if (s < nk) issue_stage(issued = s);
    }
    cur = nxt;
    w = next;
    scale_buf ^= 1;
  }
}

template <int BM, int BN, int SBK, int NSTAGE, class T, int NW = 8>
constexpr int lds_bytes() {
  if constexpr (ablk_mode<BM, BN, SBK, NSTAGE, NW, T>())
    return 2 * BM * 2 * SBK * T::kElem + MGG_ABLK_BS * SBK * BN * T::kElem;
  return NSTAGE * (BM + BN) * SBK * T::kElem;
}
// Row offsets of the derived queue's experts are kept in LDS when they fit
// beside the stages (otherwise each tile reads them from global memory).
template <int BM, int BN, int SBK, int NSTAGE, int NT, class T>
constexpr bool offsets_in_lds() {
  return lds_bytes<BM, BN, SBK, NSTAGE, T, NT / 64>() + 2 * 4 * (kMaxLdsExpertsGemm + 1) + 4 * NT + 256 +
             (T::kScaled ? 8 * (BM + BN) : 0) <=
         160 * 1024;
}

// NW waves per workgroup (4: one per SIMD; 8: two per SIMD, so one wave's
// memory and barrier stalls are filled by the other's MFMAs).  Waves form a
// 2 x NW/2 grid over the tile.
template <int BM, int BN, int SBK, int NSTAGE, int NW, class T, int EPI>
__global__ __attribute__((amdgpu_flat_work_group_size(NW * 64, NW * 64),
                          amdgpu_waves_per_eu(NW / 4, NW / 4))) void
grouped_gemm_kernel(GemmParams p) {
  static_assert(lds_bytes<BM, BN, SBK, NSTAGE, T, NW>() <= 144 * 1024, "LDS stages exceed the budget");
  constexpr int NT = NW * 64;
  constexpr bool kOffsLds = offsets_in_lds<BM, BN, SBK, NSTAGE, NT, T>();
  __shared__ __attribute__((aligned(1024))) uint8_t lds[lds_bytes<BM, BN, SBK, NSTAGE, T, NW>()];
  __shared__ int32_t s_prefix[kMaxLdsExpertsGemm + 1];
  __shared__ int32_t s_offs[kOffsLds ? kMaxLdsExpertsGemm + 1 : 1];
  __shared__ int32_t s_scan[NT];
  __shared__ int32_t s_item[2];  // [0] ticket broadcast, [1] split-tile meeting
  __shared__ float s_scale[T::kScaled ? 2 * (BM + BN) : 1];

  const int G = gridDim.x;
  const int n_tiles = (int)((p.n + BN - 1) / BN);
  // Clock probe: wave 0 of workgroups 0-7 (one per XCD) counts the shader
  // clock ticks (s_memtime) of its lifetime, which spans the launch; so few
  // readers and atomics leave the launch they measure unchanged.  (The
  // 100 MHz reference counter, s_memrealtime, is slow enough to lengthen the
  // launch, so the caller times the launch with events instead.)
  const bool probe = p.clock_probe != nullptr && blockIdx.x < 8 && threadIdx.x < 64;
  unsigned long long clk0 = 0;
  if (probe) clk0 = __builtin_amdgcn_s_memtime();

  // The work_counter's report tile differs from the compute tile when the
  // caller asked for another tile than the one that runs (the queue length it
  // reports is the requested tile's, as the reference's counter is).
  const bool rep_other =
      p.atomic && p.report != nullptr && (p.report_bm != BM || p.report_bn != BN);
  const int rep_tiles = rep_other ? (int)((p.n + p.report_bn - 1) / p.report_bn) : 0;
  int32_t w_report = 0;
  int32_t W;
  if (p.num_work >= 0) {
    W = p.num_work;
    w_report = rep_other ? queue_length<NT>(p, p.report_bm, rep_tiles, s_scan) : W;
  } else {
    W = derive_prefix<BM, NT>(p, n_tiles, s_prefix, kOffsLds ? s_offs : nullptr, s_scan,
                              rep_tiles, &w_report);
  }
  if (W == 0) {
    // No ticket is drawn: the counter word is handed on to the next launch
    // as the last ticket would have left it.
    if (p.atomic && blockIdx.x == 0 && threadIdx.x == 0)
      __hip_atomic_store(p.counter, (unsigned long long)p.next_epoch << 32, __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_AGENT);
    zero_fill<(EPI & kEpiOddN) != 0>(p, (EPI & 3) == kEpiSwiglu ? p.n / 2 : p.n);
    return;
  }

  // XCD-aware worker numbering: workgroup b runs on XCD b % 8, so giving the
  // 8 XCDs contiguous worker ranges makes each round's consecutive queue
  // items (same expert, same tile_m) share one XCD's L2.
  int v = blockIdx.x;
  if (p.remap_xcd && (G & 7) == 0) v = (blockIdx.x & 7) * (G >> 3) + (blockIdx.x >> 3);

  // Striped: items v, v+G, v+2G, ...  Atomic: worker v's first item is v
  // (the first G items need no ticket and start in the striped schedule's
  // XCD-aware placement), then tickets t of the global counter stand for
  // items G + t; a worker stops at its first ticket past the queue.
  const int32_t first = v;
  run_worker<BM, BN, SBK, NSTAGE, NW, T, EPI>(p, W, w_report, first, n_tiles, s_prefix,
                                         (kOffsLds && p.num_work < 0) ? s_offs : nullptr,
                                         s_item, lds, s_scale);
  if (probe) {
    const unsigned long long clk1 = __builtin_amdgcn_s_memtime();
    if (threadIdx.x == 0) {
      atomicAdd(p.clock_probe, clk1 - clk0);
      atomicAdd(p.clock_probe + 1, 1ull);
    }
  }
}

}  // namespace
}  // namespace mgg
