// Internal declarations shared by the libmgg HIP sources (not part of the C ABI).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <string>

namespace mgg {

// Records `msg` as the calling thread's last error and returns `code`.
int set_error(int code, const std::string& msg);
// Maps a failed HIP call to MGG_ERR_HIP with the runtime's message.
int hip_error(hipError_t err, const char* what);
void clear_error();

// Largest expert count whose per-expert tile prefix fits in LDS.
constexpr int kMaxLdsExpertsGemm = 2048;
constexpr int kMaxLdsExpertsQueue = 8192;
// Dispatch layout: assignments per chunk (one histogram row each) and the
// largest expert count whose per-chunk counters fit in LDS.
constexpr int kLayoutChunk = 1024;
constexpr int kMaxLayoutExperts = 8192;

// Fused GEMM epilogues (values of MGG_EPI_* in mgg.h).
constexpr int kEpiNone = 0;
constexpr int kEpiGelu = 1;
constexpr int kEpiSwiglu = 2;
// OR'd into a kernel's epilogue template argument (never an MGG_EPI_* value):
// the instance that reads A's rows through GemmParams::a_rows.
constexpr int kEpiGather = 4;
// Likewise: the instance for odd N (C's rows end in a 2-byte store; with
// N-major 16-bit B the term of B's last element is added separately).  Even
// N runs instances without it, whose code carries none of this.
constexpr int kEpiOddN = 8;

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Launch arguments of the grouped-GEMM kernels.  Element strides; byte
// pointers so one struct serves every element type.
struct GemmParams {
  const uint16_t* a;
  const uint16_t* b;
  uint16_t* c;
  const int32_t* offsets;
  const int32_t* q_expert;  // prebuilt queue (num_work >= 0) or null
  const int32_t* q_tile_m;
  const int32_t* q_tile_n;
  // Atomic mode: the library's dequeue counter, a 64-bit word (epoch << 32) |
  // count.  A word whose epoch is not this launch's is left over from another
  // launch (any count) and is claimed afresh as count 0; the launch's last
  // ticket leaves it at (next_epoch << 32) | 0.
  unsigned long long* counter;
  int32_t* report;   // atomic mode: caller's work_counter, receives W_report + G, or null
  int64_t m;
  int64_t k;  // any K for N-major 16-bit B (A's rows are read to the next multiple of 8)
  int64_t n;
  int64_t lda;
  int64_t ldb_e;
  int64_t ldb_k;
  int64_t ldc;
  const float* a_scale;  // fp8 only: one scale per row of A
  const float* b_scale;  // fp8 only: one scale per (expert, column of B), [E, N]
  int32_t num_experts;
  int32_t num_work;  // < 0: derive the queue from the offsets on the device
  int32_t atomic;
  int32_t remap_xcd;
  uint32_t epoch;       // atomic mode: this launch's tag in the counter word and split flags
  uint32_t next_epoch;  // the tag the last ticket leaves in the counter word (the next launch's)
  // The tile whose queue length W_report the work_counter reports (W_report
  // + G): the caller's requested tile, which may differ from the tile the
  // kernel computes with; the kernel counts it from the offsets.
  int32_t report_bm;
  int32_t report_bn;
  // Measurement hook (null normally): workgroups 0-7 add the shader-clock
  // ticks (s_memtime) of their lifetimes to [0] and 1 each to [1].
  unsigned long long* clock_probe;
  // Atomic schedule with the device-derived queue: when the last round holds
  // at most a half (a quarter) as many tiles as there are workers, each of
  // those tiles is taken as 2 (4) parts of K by as many workers (null:
  // never).  split_partials holds split_slots BM x BN fp32 partial sums
  // (uncached memory, so every XCD reads what another wrote); split_flags
  // split_slots (epoch << 32 | count) words, s - 1 per tile of s parts.
  float* split_partials;
  unsigned long long* split_flags;
  int32_t split_slots;
  // Gathered A (null normally; A-block tiles with the device-derived queue
  // only): row r of A is row a_rows[r] of the [a_src_rows, K] matrix at `a`.
  // Indices outside [0, a_src_rows) read zeros.
  const int32_t* a_rows;
  int64_t a_src_rows;
};

// The clock probe buffer set by mgg_debug_set_clock_probe (null: off).
unsigned long long* clock_probe();

// Launches the grouped GEMM for one (dtype, epilogue, block_m, block_n) on
// `stream` with `workers` workgroups.  Returns MGG_OK or an error code.
int launch_grouped_gemm(int dtype, int epilogue, int block_m, int block_n, const GemmParams& p,
                        int workers, hipStream_t stream);
// The same for odd N (p.n odd), on the tiles compiled for it: 256x256 and
// 128x128, and 128x512 for 16-bit types without a fused epilogue; other
// requested tiles compute on the nearest of these.
int launch_grouped_gemm_odd(int dtype, int epilogue, int block_m, int block_n, const GemmParams& p,
                            int workers, hipStream_t stream);
// Whether a fused epilogue is compiled for this tile shape.
bool epilogue_supported(int epilogue, int block_m, int block_n);

// Writes `value` to `count` 64-bit words with a fill kernel on `stream`.
int launch_fill_u64(unsigned long long* ptr, int count, unsigned long long value, hipStream_t stream);

int launch_offsets_from_counts(const void* counts, int counts_type, int64_t num_experts,
                               void* offsets, int out_type, hipStream_t stream);

int launch_build_work_queue(const int32_t* offsets, int32_t num_experts, int64_t n_size,
                            int block_m, int block_n, int32_t* we, int32_t* wm, int32_t* wn,
                            int32_t num_work, hipStream_t stream);

// Dispatch layout (three kernels; `hist` holds layout_chunks(T*k) * E int32).
int64_t layout_chunks(int64_t assignments);
int launch_dispatch_layout(const void* topk_idx, int idx_type, int64_t num_tokens, int top_k,
                           int32_t num_experts, int32_t* counts, int32_t* offsets,
                           int32_t* slot_pos, int32_t* token_index, int32_t* row_assign,
                           int32_t* hist, hipStream_t stream);
int launch_gather_rows(const void* x, int64_t ld_x, const int32_t* token_index,
                       const int32_t* rows_ptr, int64_t rows_max, int64_t hidden, int elem_bytes,
                       void* out, int64_t ld_out, hipStream_t stream);
int launch_combine_rows(int dtype, const void* y, int64_t ld_y, const int32_t* slot_pos,
                        const float* weight, int64_t num_tokens, int top_k, int64_t hidden,
                        void* out, int64_t ld_out, hipStream_t stream);

}  // namespace mgg
