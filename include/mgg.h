/*
 * mgg.h - C ABI of the MI355X (gfx950) expert-grouped GEMM library (libmgg.so).
 *
 * Plain pointers, sizes and a HIP stream passed as void*.  No torch or C++
 * types cross this boundary and no C++ exception escapes it: every entry point
 * returns MGG_OK or an error code, and mgg_last_error() returns a message for
 * the calling thread's most recent failure.
 *
 * Device pointers are borrowed for the duration of the (asynchronous) launch
 * only; the library never frees caller memory.  All work is enqueued on the
 * given stream; nothing here synchronises the device.
 *
 * Reference interface replaced by each entry point (paths relative to the
 * Hongyu15/moe-overlap checkout):
 *   mgg_expert_offsets_from_counts -> src/triton_grouped_gemm.py:300-323
 *                                     (expert_offsets_from_recv_counts)
 *   mgg_build_work_queue           -> src/triton_grouped_gemm.py:240-297
 *                                     (_build_work_queue, device part)
 *   mgg_grouped_gemm               -> src/triton_grouped_gemm.py:326-443
 *                                     (persistent_grouped_gemm launch), with the
 *                                     tile kernels of :36-233
 *   mgg_device_cu_count            -> the `num_sms` grid size the reference
 *                                     passes by hand (:330, :375)
 *   mgg_grouped_gemm_ex            -> the expert MLP's two GEMMs with the
 *                                     activation fused in
 *                                     (src/train_moe_baseline.py:239-242)
 *   mgg_dispatch_layout            -> sort / bincount / cumsum / inv_perm of
 *                                     src/train_moe_baseline.py:219-237 (and the
 *                                     per-expert counts of DeepEP's
 *                                     csrc/kernels/layout.cu:10-121)
 *   mgg_gather_rows                -> grouped_tokens = valid_tokens[perm]
 *                                     (src/train_moe_baseline.py:224)
 *   mgg_grouped_gemm_gathered      -> that gather and the expert MLP's first
 *                                     GEMM in one launch
 *                                     (src/train_moe_baseline.py:224, :239-241)
 *   mgg_grouped_gemm_fp8           -> no counterpart: the reference rejects
 *                                     fp8 (src/triton_grouped_gemm.py:357-358);
 *                                     the fp8 config of the build's baseline
 *   mgg_combine_rows               -> out[valid] = grouped_out[inv_perm] and
 *                                     out += y * gate over the top-k slots
 *                                     (src/train_moe_baseline.py:245-246, :340-341)
 *   mgg_debug_set_dequeue_counter  -> no counterpart: a test hook (the
 *                                     reference zeroes its counter on the
 *                                     host before each launch, :379-386)
 *   mgg_debug_set_clock_probe      -> no counterpart: a measurement hook
 *   mgg_debug_counter_slots        -> no counterpart: a test hook
 *   mgg_debug_set_split_flags      -> no counterpart: a test hook (the
 *                                     reference never splits a tile)
 *   mgg_dispatch_layout_noalloc    -> no counterpart: mgg_dispatch_layout
 *                                     for callers that cannot allocate
 *   mgg_set_split_last_round,      -> no counterpart: controls of the atomic
 *   mgg_reserve_split_workspace,      schedule's split last round (the
 *   mgg_split_workspace_bytes         reference's atomic kernel, :157-233,
 *                                     takes whole items)
 */
#ifndef MGG_H_
#define MGG_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes. */
#define MGG_OK 0
#define MGG_ERR_INVALID 1     /* bad argument (shape, size, alignment, pointer) */
#define MGG_ERR_UNSUPPORTED 2 /* valid request outside what the kernels cover   */
#define MGG_ERR_HIP 3         /* HIP runtime call failed                        */

/* Element types of the GEMM operands. */
#define MGG_DTYPE_BF16 0
#define MGG_DTYPE_FP16 1
#define MGG_DTYPE_FP8_E4M3 2 /* OCP e4m3 (float8_e4m3fn) operands, BF16 output */
/* OR'd into the BF16/FP16 dtype of mgg_grouped_gemm and mgg_grouped_gemm_ex:
 * B is stored [E, N, K] with K contiguous (a linear layer's [out, in] weight,
 * passed by the reference's callers as its [E, K, N] transposed view), and
 * ldb_k is the stride between B's N rows (>= K).  Results are bitwise those
 * of the same values stored [E, K, N].  (Introduced with ABI version 3.) */
#define MGG_B_KMAJOR 0x100

/* Fused GEMM epilogues (mgg_grouped_gemm_ex). */
#define MGG_EPI_NONE 0
#define MGG_EPI_GELU 1   /* C = gelu(A @ B), erf form (torch.nn.functional.gelu) */
#define MGG_EPI_SWIGLU 2 /* C = silu(A @ Bgate) * (A @ Bup), B columns interleaved */

/* Integer types of the per-expert count vector. */
#define MGG_INT32 0
#define MGG_INT64 1

/* Library ABI version (bumped on any signature change). */
int mgg_abi_version(void);

/* Message for the calling thread's most recent failed call ("" if none). */
const char* mgg_last_error(void);

/* Number of compute units of HIP device `device` (256 on MI355X). */
int mgg_device_cu_count(int device, int* cu_count);

/*
 * offsets[0] = 0, offsets[i+1] = offsets[i] + (int32)counts[i], i < E.
 * `counts` is int32 or int64 (counts_type) on the device; each count is first
 * narrowed to int32 (two's-complement wrap), as `.to(torch.int32)` does.
 * `offsets` is int32 (out_type MGG_INT32, sums wrap modulo 2^32) or int64
 * (MGG_INT64, exact), length E+1.  E == 0 writes offsets = [0].
 */
int mgg_expert_offsets_from_counts(const void* counts, int counts_type, int64_t num_experts,
                                   void* offsets, int out_type, void* stream);

/*
 * Fill the tile work queue for `expert_offsets` (int32, length E+1, device):
 * for each expert e in order, count_e = max(off[e+1]-off[e], 0),
 * tm_e = ceil(count_e / block_m), tn = ceil(n_size / block_n), and items
 * (e, tm, tn) for tm < tm_e, tn < tn in row-major order (tile_n fastest).
 * `num_work` must equal sum_e tm_e * tn (the caller computes it); the three
 * int32 output arrays have num_work entries.  E must be <= 8192.
 */
int mgg_build_work_queue(const int32_t* expert_offsets, int64_t num_experts, int64_t n_size,
                         int block_m, int block_n, int32_t* work_expert, int32_t* work_tile_m,
                         int32_t* work_tile_n, int64_t num_work, void* stream);

/*
 * Host-memory variants of the two builders above, for counts/offsets that
 * live in CPU memory (the reference's torch ops accept CPU tensors too).
 * Same arguments and results; they run synchronously on the calling thread.
 */
int mgg_expert_offsets_from_counts_host(const void* counts, int counts_type, int64_t num_experts,
                                        void* offsets, int out_type);
int mgg_build_work_queue_host(const int64_t* expert_offsets, int64_t num_experts, int64_t n_size,
                              int block_m, int block_n, int32_t* work_expert,
                              int32_t* work_tile_m, int32_t* work_tile_n, int64_t num_work);

/*
 * Persistent grouped GEMM:  C[off[e]+i, :] = A[off[e]+i, :] @ B[e]  for
 * 0 <= i < max(off[e+1]-off[e], 0), every expert e, fp32 accumulation, output
 * in the input dtype (round to nearest even).
 *
 *   a  [M, K]     row stride lda   (elements; unit inner stride)
 *   b  [E, K, N]  expert stride ldb_e, row stride ldb_k (unit inner stride)
 *   c  [M, N]     row stride ldc
 *   expert_offsets  int32 [E+1] on the device
 *
 * Work items are BLOCK_M x BLOCK_N output tiles.
 * work_expert/work_tile_m/work_tile_n (num_work entries, from
 * mgg_build_work_queue) are used, in their order, when num_work >= 0; with
 * num_work < 0 and null queue pointers, the kernel derives the same tiles
 * from the offsets on the device (no host round trip), ordered expert by
 * expert and, within an expert, in groups of 4 m-tiles taken n-tile by
 * n-tile (the group's m-tiles consecutive), so that each XCD's share of a
 * round spans few A and B blocks.  A tile's sums do not depend on the order.
 *
 * num_workers persistent workgroups are launched (<= 0 means one per CU).
 * use_atomic_queue = 0: worker w takes items w, w+G, w+2G, ... (workers are
 * numbered so that each XCD owns a contiguous slice of every round).
 * use_atomic_queue = 1: workers take the next item with an atomic add on a
 * 64-bit counter word (every worker's first item, and with the
 * device-derived queue and at least 2G tiles its items of every whole round,
 * are its stripes, taken without a ticket; tickets serve the tail).  The word is owned by the library: one per (device, stream) for
 * direct launches, and one per (capture, stream) for launches captured into
 * a HIP graph (so graph replays never share a word with other launches; the
 * word is released when the graph is destroyed).  The words live in a
 * file-scope device array (no allocation; at most 4096 held at once per
 * device).  Each launch tags the word with its epoch (the next in the
 * word's sequence) and claims whatever other value it finds there, so a
 * word left dirty by a launch that did not finish never drops or repeats
 * tiles; the launch's last ticket leaves the word tagged for the next one.
 * Graph replays of one captured launch are ordered on their stream; one
 * graph replayed on two streams at once would share its word and race.
 * If work_counter is non-null (device int32) it receives W + G, the value
 * the reference's counter ends at (:379-416: each worker over-fetches once),
 * where W is the queue length of the report tile, report_block_m x
 * report_block_n (<= 0: block_m x block_n): the tile the caller asked for
 * when the library computes with another.  With an empty queue it is left
 * untouched, as there.  Calls on one stream are ordered; calls on
 * different streams use different counters.
 *
 * If the queue is empty, C is zero-filled; with K == 0 the covered rows are
 * zeros (A and B and their strides are not read).  Rows of C not covered by
 * any expert range are left unwritten.  Supported: dtype BF16/FP16,
 * block_m, block_n in {64, 128, 256} or 128 x 512, any N (B's and C's rows
 * are read and written at any 2-byte alignment; the last chunk of a C row
 * is stored by pairs and, for odd N, one 2-byte store), lda (and ldb_k of
 * K-major B) a multiple of 8 elements, any ldb_k of N-major B, ldb_e and
 * ldc, 16-byte aligned base pointers, E <= 2048 when the queue is derived
 * on the device.  B must span its view: (E-1)*ldb_e + (K-1)*ldb_k + N
 * elements for N-major B (ldb_e may be 0: every expert shares one B).
 * K % 8 == 0 for K-major B; with N-major B any K:
 * B's rows at and past K are never read (they count as zeros), while A is
 * read up to the next multiple of 8, so lda must cover it and A's elements
 * in those columns must be finite (they are multiplied by zeros; the drop-in
 * makes them zeros).
 * (ABI version 4 added report_block_m, report_block_n; version 6 any K for
 * N-major B; version 7 the split controls, per-capture counter words and
 * any even N; version 8 odd N and any B and C strides.)
 */
int mgg_grouped_gemm(int dtype, const void* a, const void* b, void* c,
                     const int32_t* expert_offsets, int64_t m_size, int64_t k_size, int64_t n_size,
                     int64_t num_experts, int64_t lda, int64_t ldb_e, int64_t ldb_k, int64_t ldc,
                     const int32_t* work_expert, const int32_t* work_tile_m,
                     const int32_t* work_tile_n, int64_t num_work, int block_m, int block_n,
                     int num_workers, int use_atomic_queue, int32_t* work_counter,
                     int report_block_m, int report_block_n, void* stream);

/*
 * mgg_grouped_gemm with a fused element-wise epilogue.  Same arguments and
 * semantics otherwise (the queue is derived on the device when num_work < 0,
 * or read from work_expert/work_tile_m/work_tile_n, e.g. above 2048 experts).
 *   MGG_EPI_GELU:   C[r, n] = gelu(sum_k A[r, k] B[e, k, n]) (fp32, then rounded).
 *   MGG_EPI_SWIGLU: B's N columns hold gate and up projections interleaved in
 *                   groups of 64: columns 64q .. 64q+31 are gate outputs
 *                   32q .. 32q+31, columns 64q+32 .. 64q+63 the up outputs of
 *                   the same indices.  C has N/2 columns:
 *                   C[r, f] = silu(gate[r, f]) * up[r, f].  N % 64 == 0.
 * Fused epilogues are compiled for block_m == block_n in {128, 256}.
 * (Introduced with ABI version 2; version 4 added the queue and report-tile
 * arguments.)
 */
int mgg_grouped_gemm_ex(int dtype, int epilogue, const void* a, const void* b, void* c,
                        const int32_t* expert_offsets, int64_t m_size, int64_t k_size,
                        int64_t n_size, int64_t num_experts, int64_t lda, int64_t ldb_e,
                        int64_t ldb_k, int64_t ldc, const int32_t* work_expert,
                        const int32_t* work_tile_m, const int32_t* work_tile_n, int64_t num_work,
                        int block_m, int block_n, int num_workers, int use_atomic_queue,
                        int32_t* work_counter, int report_block_m, int report_block_n,
                        void* stream);

/*
 * mgg_grouped_gemm_ex with A's rows gathered: row r of A (r < m_size, in the
 * expert-grouped order of expert_offsets) is row a_rows[r] of `a`, a
 * [a_src_rows, k_size] matrix with row stride lda.  a_rows is int32 on the
 * device; only the rows of the experts' ranges are read, and an index outside
 * [0, a_src_rows) reads a row of zeros.  Results are bitwise those of
 * mgg_grouped_gemm_ex on the gathered matrix (same tiles, same schedule).
 * Covers 16-bit operands with N-major B, block_m == block_n == 256 and the
 * device-derived queue (at most 2048 experts); every epilogue.  The
 * work_counter is not offered (no caller-visible queue).  (Introduced with ABI
 * version 6.)
 */
int mgg_grouped_gemm_gathered(int dtype, int epilogue, const void* a, const int32_t* a_rows,
                              int64_t a_src_rows, const void* b, void* c,
                              const int32_t* expert_offsets, int64_t m_size, int64_t k_size,
                              int64_t n_size, int64_t num_experts, int64_t lda, int64_t ldb_e,
                              int64_t ldb_k, int64_t ldc, int num_workers, int use_atomic_queue,
                              void* stream);

/*
 * fp8 grouped GEMM with per-token and per-channel scales:
 *   C[r, n] = a_scale[r] * b_scale[e, n] * sum_k A[r, k] * B[e, n, k]
 * for rows r of expert e's range, fp32 accumulation, BF16 output.
 *   a  [M, K]     OCP e4m3 bytes, row stride lda
 *   b  [E, N, K]  OCP e4m3 bytes, K contiguous (the [out, in] layout of a
 *                 linear layer's weight), expert stride ldb_e, row stride ldb_n
 *   a_scale [M], b_scale [E, N] (row stride N): fp32 on the device
 *   c  [M, N]     BF16, row stride ldc
 * Queue (derived on the device, or prebuilt), schedules, work_counter and
 * empty-queue behaviour as in mgg_grouped_gemm.  Tiles 256x256, 256x128,
 * 192x128 and 128x128; K, lda, ldb_n, ldb_e multiples of 16; any N and
 * ldc.
 * (Introduced with ABI version 2; version 4 added the queue and report-tile
 * arguments; version 8 odd N and any ldc.)
 */
int mgg_grouped_gemm_fp8(const void* a, const void* b, void* c, const int32_t* expert_offsets,
                         const float* a_scale, const float* b_scale, int64_t m_size,
                         int64_t k_size, int64_t n_size, int64_t num_experts, int64_t lda,
                         int64_t ldb_e, int64_t ldb_n, int64_t ldc, const int32_t* work_expert,
                         const int32_t* work_tile_m, const int32_t* work_tile_n,
                         int64_t num_work, int block_m, int block_n, int num_workers,
                         int use_atomic_queue, int32_t* work_counter, int report_block_m,
                         int report_block_n, void* stream);

/*
 * Test hook, no counterpart in the reference: writes `value` into the atomic
 * queue's counter word of direct launches on `stream` (current device), the
 * state a launch that did not finish could leave behind, so tests can check
 * that the next launch still computes every tile.  Enqueued on `stream`.
 */
int mgg_debug_set_dequeue_counter(uint64_t value, void* stream);

/*
 * Test hook, no counterpart in the reference: *held = the number of counter
 * words of `device` now assigned to a stream or to a live graph capture
 * (words of destroyed graphs are free again).
 */
int mgg_debug_counter_slots(int device, int* held);

/*
 * Measurement hook, no counterpart in the reference: while `probe` (device
 * memory, two uint64, caller-zeroed) is set, every grouped-GEMM launch adds,
 * for each of its first eight workgroups, the shader-clock ticks (s_memtime)
 * of its lifetime to probe[0] and 1 to probe[1]; probe[0] / probe[1] over the
 * launch time (e.g. from HIP events) is the shader clock the kernel ran at.
 * Null turns it off (the default).  Process-wide.
 */
int mgg_debug_set_clock_probe(uint64_t* probe);

/*
 * Test hook, no counterpart in the reference: writes `value` into every
 * split-tile flag word of atomic launches on `stream` (current device), the
 * state a launch that did not finish could leave behind.  An atomic launch
 * whose last round holds at most a quarter (a half) as many tiles as workers
 * takes each of those tiles as 4 (2) parts of K, which meet pairwise through
 * these words.  Fails with
 * MGG_ERR_INVALID before the stream's first atomic launch (no words yet).
 * Enqueued on `stream`.
 */
int mgg_debug_set_split_flags(uint64_t value, void* stream);

/*
 * The atomic schedule's split last round, no counterpart in the reference
 * (its atomic kernel takes whole items).  With the device-derived queue, an
 * atomic launch whose last round holds at most a quarter (a third, a half)
 * as many tiles as workers takes each of those tiles as 4 (3, 2) parts of K
 * (each part of an even cut at least 1024 deep in K, so K >= 2048 for
 * halves, 3072 for thirds, 4096 for quarters; twice that for fp8); the
 * parts'
 * fp32 sums meet in a per-(device, stream) workspace of one 256 x 256 fp32
 * slot per CU (64 MiB on a 256-CU device) plus one flag word per CU.  The
 * sums then round differently in the last bits from the unsplit tile
 * (striped, graph-captured, or split-off launches of the same call).
 *
 * mgg_set_split_last_round(0) turns splitting off process-wide (every tile
 * whole, bitwise the striped schedule's results); 1 turns it back on (the
 * default).  mgg_reserve_split_workspace makes the workspace of `stream` on
 * the current device now, so no launch allocates it (otherwise the first
 * atomic launch on the stream that could split does); it is never freed,
 * and it cannot be made under graph capture (MGG_ERR_INVALID).  At most 16
 * streams per device get one; launches on further streams, and launches
 * under graph capture, take every tile whole.
 * mgg_split_workspace_bytes reports the bytes held for `stream` (0: none).
 */
int mgg_set_split_last_round(int enabled);
int mgg_reserve_split_workspace(void* stream);
int mgg_split_workspace_bytes(void* stream, int64_t* bytes);

/*
 * Dispatch layout of T tokens routed to top_k experts each (one GPU's share):
 *   topk_idx  [T, top_k] int32 or int64 (idx_type), row-major, on the device;
 *             entries outside [0, E) (e.g. -1) are masked assignments.
 * Outputs (device, int32):
 *   counts[E]            assignments per expert;
 *   offsets[E+1]         exclusive prefix of counts (offsets[E] = valid total);
 *   slot_position[T*k]   row of assignment a = t*top_k + j in the expert-major
 *                        order (stable: by a within an expert), -1 if masked;
 *   token_index[T*k]     for rows p < offsets[E]: the token of row p;
 *   row_assignment[T*k]  for rows p < offsets[E]: the assignment a of row p.
 * workspace: device memory of mgg_dispatch_layout_workspace_bytes() bytes
 * (overwritten).  E <= 8192, T*top_k < 2^31.  No host synchronisation.
 */
int64_t mgg_dispatch_layout_workspace_bytes(int64_t num_tokens, int top_k, int64_t num_experts);
int mgg_dispatch_layout(const void* topk_idx, int idx_type, int64_t num_tokens, int top_k,
                        int64_t num_experts, int32_t* counts, int32_t* offsets,
                        int32_t* slot_position, int32_t* token_index, int32_t* row_assignment,
                        void* workspace, int64_t workspace_bytes, void* stream);

/*
 * mgg_dispatch_layout without a workspace argument, for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  No counterpart in the reference.  The
 * workspace is a 1 MiB array inside the library (one per device, held until
 * the process ends): layouts whose mgg_dispatch_layout_workspace_bytes()
 * exceeds 1 MiB (e.g. more than 262144 assignments over 1024 experts) are
 * rejected with MGG_ERR_UNSUPPORTED.  No memory is allocated.  Every call
 * on one device shares that array: calls that overlap on one device (on
 * unordered streams) race.  Results are those of mgg_dispatch_layout.
 */
int mgg_dispatch_layout_noalloc(const void* topk_idx, int idx_type, int64_t num_tokens, int top_k,
                                int64_t num_experts, int32_t* counts, int32_t* offsets,
                                int32_t* slot_position, int32_t* token_index,
                                int32_t* row_assignment, void* stream);

/*
 * out[p, :] = x[token_index[p], :] for p < rows, rows = *num_rows (device
 * int32, e.g. offsets + E from mgg_dispatch_layout) clamped to max_rows, or
 * max_rows when num_rows is null.  Rows of `hidden` BF16/FP16 elements with
 * leading dimensions ld_x, ld_out.
 */
int mgg_gather_rows(int dtype, const void* x, int64_t ld_x, const int32_t* token_index,
                    const int32_t* num_rows, int64_t max_rows, int64_t hidden, void* out,
                    int64_t ld_out, void* stream);

/*
 * out[t, :] = sum_{j < top_k, slot_position[t*top_k+j] >= 0}
 *             weights[t*top_k+j] * y[slot_position[t*top_k+j], :]
 * for t < num_tokens: fp32 accumulation in slot order, one rounding to the
 * output type (BF16/FP16, same as y).  weights: fp32 [T, top_k] on the device.
 */
int mgg_combine_rows(int dtype, const void* y, int64_t ld_y, const int32_t* slot_position,
                     const float* weights, int64_t num_tokens, int top_k, int64_t hidden,
                     void* out, int64_t ld_out, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* MGG_H_ */
