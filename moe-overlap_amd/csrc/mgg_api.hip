// extern "C" entry points of libmgg.so (declared in include/mgg.h): argument
// validation, library-owned dequeue counters, and the launches.  No C++
// exception crosses this boundary; failures return a status code and leave a
// message for mgg_last_error().
#include <algorithm>
#include <atomic>
#include <deque>
#include <map>
#include <mutex>
#include <string>
#include <utility>
#include <vector>

#include <hip/hip_ext.h>

#include "mgg.h"
#include "mgg_internal.h"

namespace mgg {

// Dequeue counters of the atomic schedule: one 64-bit word per slot, in a
// file-scope device array (each device holds its own copy for the life of
// the process), so no entry point allocates memory.  A word holds (epoch <<
// 32) | count; each launch carries a fresh epoch and claims whatever value
// it finds (see first_ticket in mgg_gemm.hip), so a launch that did not run
// to its end cannot leave a count that the next launch trusts.
constexpr int kCounterSlots = 4096;
__device__ __align__(256) unsigned long long counter_pool[kCounterSlots];

// Workspace of mgg_dispatch_layout_noalloc: the per-chunk expert histogram
// (layout_chunks(T * top_k) * E int32, every entry written by the count pass
// before any pass reads it, so nothing needs clearing), at most
// kScratchBytes.  Each device holds its own copy for the life of the
// process; every call on a device shares it, so such calls must not overlap
// on one device (one stream, or ordered streams).
constexpr int64_t kScratchBytes = (int64_t)1 << 20;
__device__ __align__(256) int32_t scratch[kScratchBytes / sizeof(int32_t)];

namespace {

thread_local std::string g_last_error;

std::atomic<unsigned long long*> g_clock_probe{nullptr};
std::atomic<int> g_split_enabled{1};

// Epoch of the seq-th launch on a counter slot: distinct for 2^32 launches,
// and never 0, the value every word starts at and the likeliest junk.
uint32_t epoch_of(uint32_t seq) {
  const uint32_t e = (seq + 1u) * 0x9E3779B1u;
  return e != 0 ? e : 1u;
}

// Counter slots.  Direct launches on one (device, stream) share a slot (they
// run in stream order), and each launch tags it with the slot's next epoch
// in sequence and leaves it tagged with the one after, so the next launch
// finds its own epoch there.  Launches captured into a graph on one stream in
// one capture share a slot of their own with one fixed epoch (they run in
// order within the graph, and every replay starts where the last one ended);
// the slot returns to the device's free list when the graph is destroyed
// (a user object the graph holds), and freed slots are reused oldest first,
// after every never-used slot.
struct CaptureKey {
  int device;
  unsigned long long capture_id;
  hipStream_t stream;
  bool operator<(const CaptureKey& o) const {
    if (device != o.device) return device < o.device;
    if (capture_id != o.capture_id) return capture_id < o.capture_id;
    return stream < o.stream;
  }
};
struct CapturedSlot {
  int slot;
  uint32_t epoch;
};
struct CounterSlots {
  std::mutex mu;
  std::map<std::pair<int, hipStream_t>, int> by_stream;
  std::map<CaptureKey, CapturedSlot> by_capture;
  std::vector<unsigned long long*> base;      // per device: counter_pool's address there
  std::vector<int> used;                      // per device: slots ever handed out
  std::vector<std::deque<int>> freed;         // per device: released slots, oldest first
  std::vector<std::vector<uint32_t>> seq;     // per device, per slot: launches so far
};
CounterSlots g_slots;

int pool_base(int device, unsigned long long** out) {
  if ((int)g_slots.base.size() <= device) {
    g_slots.base.resize(device + 1, nullptr);
    g_slots.used.resize(device + 1, 0);
    g_slots.freed.resize(device + 1);
    g_slots.seq.resize(device + 1);
  }
  if (g_slots.base[device] == nullptr) {
    void* ptr = nullptr;
    const hipError_t err = hipGetSymbolAddress(&ptr, HIP_SYMBOL(counter_pool));
    if (err != hipSuccess) return hip_error(err, "hipGetSymbolAddress(counter_pool)");
    g_slots.base[device] = static_cast<unsigned long long*>(ptr);
    g_slots.seq[device].assign(kCounterSlots, 0u);
  }
  *out = g_slots.base[device];
  return MGG_OK;
}

// A slot for a new owner (g_slots.mu held): never-used slots first, then the
// longest-released one; -1 when every slot is held.
int take_slot(int device) {
  if (g_slots.used[device] < kCounterSlots) return g_slots.used[device]++;
  if (!g_slots.freed[device].empty()) {
    const int s = g_slots.freed[device].front();
    g_slots.freed[device].pop_front();
    return s;
  }
  return -1;
}

// Destructor of the user object a capturing graph holds: its slot is free.
void release_captured_slot(void* arg) {
  CaptureKey* key = static_cast<CaptureKey*>(arg);
  {
    std::lock_guard<std::mutex> lock(g_slots.mu);
    auto it = g_slots.by_capture.find(*key);
    if (it != g_slots.by_capture.end()) {
      g_slots.freed[key->device].push_back(it->second.slot);
      g_slots.by_capture.erase(it);
    }
  }
  delete key;
}

// scratch's device address on the current device, looked up once per device
// (the array's host-side name is only a stand-in for it).
std::mutex g_scratch_mu;
std::vector<int32_t*> g_scratch_ptr;

int scratch_for_current_device(int32_t** out) {
  int device = 0;
  hipError_t err = hipGetDevice(&device);
  if (err != hipSuccess) return hip_error(err, "hipGetDevice");
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if ((int)g_scratch_ptr.size() <= device) g_scratch_ptr.resize(device + 1, nullptr);
  if (g_scratch_ptr[device] == nullptr) {
    void* ptr = nullptr;
    err = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (err != hipSuccess) return hip_error(err, "hipGetSymbolAddress(scratch)");
    g_scratch_ptr[device] = static_cast<int32_t*>(ptr);
  }
  *out = g_scratch_ptr[device];
  return MGG_OK;
}

// The counter word for a launch on `stream` (current device), the launch's
// epoch and the epoch it leaves in the word for the slot's next launch.
// `count_launch` false: only the word (the debug hook).
int counter_for(hipStream_t stream, unsigned long long** out, uint32_t* epoch, uint32_t* next,
                bool count_launch = true) {
  int device = 0;
  hipError_t err = hipGetDevice(&device);
  if (err != hipSuccess) return hip_error(err, "hipGetDevice");
  hipStreamCaptureStatus capture = hipStreamCaptureStatusNone;
  unsigned long long capture_id = 0;
  hipGraph_t graph = nullptr;
  if (stream != nullptr) {
    const hipGraphNode_t* deps = nullptr;
    size_t num_deps = 0;
    err = hipStreamGetCaptureInfo_v2(stream, &capture, &capture_id, &graph, &deps, &num_deps);
    if (err != hipSuccess) return hip_error(err, "hipStreamGetCaptureInfo_v2");
  }
  unsigned long long* base = nullptr;
  if (capture == hipStreamCaptureStatusNone || !count_launch) {
    std::lock_guard<std::mutex> lock(g_slots.mu);
    int rc = pool_base(device, &base);
    if (rc != MGG_OK) return rc;
    const auto key = std::make_pair(device, stream);
    auto it = g_slots.by_stream.find(key);
    int slot;
    if (it != g_slots.by_stream.end()) {
      slot = it->second;
    } else {
      slot = take_slot(device);
      if (slot < 0)
        return set_error(MGG_ERR_UNSUPPORTED,
                         "atomic queue: more than 4096 streams and live captures on one device");
      g_slots.by_stream.emplace(key, slot);
    }
    *out = base + slot;
    if (count_launch) {
      uint32_t& s = g_slots.seq[device][slot];
      *epoch = epoch_of(s);
      *next = epoch_of(s + 1);
      ++s;
    }
    return MGG_OK;
  }
  const CaptureKey key{device, capture_id, stream};
  bool fresh = false;
  int slot = -1;
  {
    std::lock_guard<std::mutex> lock(g_slots.mu);
    int rc = pool_base(device, &base);
    if (rc != MGG_OK) return rc;
    auto it = g_slots.by_capture.find(key);
    if (it != g_slots.by_capture.end()) {
      *out = base + it->second.slot;
      *epoch = *next = it->second.epoch;
      return MGG_OK;
    }
    slot = take_slot(device);
    if (slot < 0)
      return set_error(MGG_ERR_UNSUPPORTED,
                       "atomic queue: more than 4096 streams and live captures on one device");
    // The slot's next epoch in sequence: different from whatever its last
    // owner left in the word.
    const uint32_t e = epoch_of(g_slots.seq[device][slot]++);
    g_slots.by_capture.emplace(key, CapturedSlot{slot, e});
    *out = base + slot;
    *epoch = *next = e;
    fresh = true;
  }
  if (fresh && graph != nullptr) {
    // The graph holds the only reference: its destruction frees the slot.
    // Without a user object the slot stays held (the launch still runs).
    // (If the graph cannot take the object, it and the slot stay held.)
    CaptureKey* arg = new CaptureKey(key);
    hipUserObject_t obj = nullptr;
    if (hipUserObjectCreate(&obj, arg, release_captured_slot, 1, hipUserObjectNoDestructorSync) !=
        hipSuccess) {
      (void)hipGetLastError();
      delete arg;
    } else if (hipGraphRetainUserObject(graph, obj, 1, hipGraphUserObjectMove) != hipSuccess) {
      (void)hipGetLastError();
    }
  }
  return MGG_OK;
}

// Split-tile workspaces of the atomic schedule, one per (device, stream):
// fp32 partial sums in uncached memory (a part written on one XCD is read on
// another, and no cache level may hold a stale copy) and zeroed flag words,
// one slot and one flag word per work item of a split tile (a tile of s parts
// uses s slots and s - 1 flags).  A split never has more work items than the
// launch has workers and happens only when they fit in the slots, so the
// workspace holds one 256 x 256 slot (the largest tile) per CU and no
// more: 64 MiB on a 256-CU device, whatever the launch's worker count or
// tile.  It is made once, by mgg_reserve_split_workspace or the stream's
// first atomic launch that could split, and never replaced or freed
// (uncached memory a kernel has read must stay allocated until the process
// ends).  A launch under graph capture gets none (it takes every tile
// whole), so capture never allocates.  At most kMaxSplitSpaces streams per
// device get one; launches on further streams take every tile whole.
constexpr int kMaxSplitSpaces = 16;
constexpr int64_t kSplitSlotBytes = 256 * 256 * 4;
struct SplitSpace {
  float* partials = nullptr;
  unsigned long long* flags = nullptr;
  int64_t bytes = 0;  // of partials
  int64_t flag_words = 0;
};
std::mutex g_split_mu;
std::map<std::pair<int, hipStream_t>, SplitSpace> g_split;

// The workspace of (current device, stream), made if `create` and possible;
// *out is null when there is none.
int split_space(hipStream_t stream, bool create, const SplitSpace** out) {
  *out = nullptr;
  int device = 0;
  hipError_t err = hipGetDevice(&device);
  if (err != hipSuccess) return hip_error(err, "hipGetDevice");
  const auto key = std::make_pair(device, stream);
  std::lock_guard<std::mutex> lock(g_split_mu);
  auto it = g_split.find(key);
  if (it != g_split.end()) {
    *out = &it->second;
    return MGG_OK;
  }
  if (!create) return MGG_OK;
  int on_device = 0;
  for (const auto& kv : g_split) on_device += kv.first.first == device ? 1 : 0;
  if (on_device >= kMaxSplitSpaces) return MGG_OK;
  int cus = 0;
  err = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device);
  if (err != hipSuccess) return hip_error(err, "hipDeviceGetAttribute(MultiprocessorCount)");
  const int64_t words = cus > 0 ? cus : 1;
  const int64_t bytes = words * kSplitSlotBytes;
  void* partials = nullptr;
  void* flags = nullptr;
  if (hipExtMallocWithFlags(&partials, (size_t)bytes, hipDeviceMallocUncached) != hipSuccess) {
    (void)hipGetLastError();  // no workspace: launches take every tile whole
    return MGG_OK;
  }
  if (hipMalloc(&flags, (size_t)words * 8) != hipSuccess) {
    (void)hipGetLastError();  // (the uncached block stays allocated, unused)
    return MGG_OK;
  }
  err = hipMemsetAsync(flags, 0, (size_t)words * 8, stream);
  if (err != hipSuccess) return hip_error(err, "hipMemsetAsync(split flags)");
  SplitSpace& sp = g_split[key];
  sp.partials = static_cast<float*>(partials);
  sp.flags = static_cast<unsigned long long*>(flags);
  sp.bytes = bytes;
  sp.flag_words = words;
  *out = &sp;
  return MGG_OK;
}

// Sets p's split fields for a launch of BM x BN tiles on `stream`, or leaves
// them null (every tile whole): splitting turned off, graph capture, or no
// workspace to be had.
int split_space_for(hipStream_t stream, int block_m, int block_n, GemmParams* p) {
  if (!g_split_enabled.load()) return MGG_OK;
  if (stream != nullptr) {
    hipStreamCaptureStatus capture = hipStreamCaptureStatusNone;
    const hipError_t err = hipStreamIsCapturing(stream, &capture);
    if (err != hipSuccess) return hip_error(err, "hipStreamIsCapturing");
    if (capture != hipStreamCaptureStatusNone) return MGG_OK;
  }
  const SplitSpace* sp = nullptr;
  const int rc = split_space(stream, true, &sp);
  if (rc != MGG_OK || sp == nullptr) return rc;
  const int64_t slot_bytes = (int64_t)block_m * block_n * 4;
  p->split_partials = sp->partials;
  p->split_flags = sp->flags;
  p->split_slots = (int32_t)std::min<int64_t>(sp->bytes / slot_bytes, sp->flag_words);
  return MGG_OK;
}

}  // namespace

unsigned long long* clock_probe() { return g_clock_probe.load(); }

int set_error(int code, const std::string& msg) {
  g_last_error = msg;
  return code;
}

int hip_error(hipError_t err, const char* what) {
  if (err == hipSuccess) return MGG_OK;
  return set_error(MGG_ERR_HIP, std::string(what) + ": " + hipGetErrorString(err));
}

void clear_error() { g_last_error.clear(); }

}  // namespace mgg

using mgg::set_error;

extern "C" {

int mgg_abi_version(void) { return 8; }

const char* mgg_last_error(void) { return mgg::g_last_error.c_str(); }

int mgg_device_cu_count(int device, int* cu_count) {
  mgg::clear_error();
  if (cu_count == nullptr) return set_error(MGG_ERR_INVALID, "cu_count is null");
  int n = 0;
  const hipError_t err = hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, device);
  if (err != hipSuccess) return mgg::hip_error(err, "hipDeviceGetAttribute(MultiprocessorCount)");
  *cu_count = n;
  return MGG_OK;
}

int mgg_expert_offsets_from_counts(const void* counts, int counts_type, int64_t num_experts,
                                   void* offsets, int out_type, void* stream) {
  mgg::clear_error();
  if (num_experts < 0) return set_error(MGG_ERR_INVALID, "num_experts must be >= 0");
  if (offsets == nullptr) return set_error(MGG_ERR_INVALID, "offsets is null");
  if (num_experts > 0 && counts == nullptr) return set_error(MGG_ERR_INVALID, "counts is null");
  return mgg::launch_offsets_from_counts(counts, counts_type, num_experts, offsets, out_type,
                                         static_cast<hipStream_t>(stream));
}

int mgg_build_work_queue(const int32_t* expert_offsets, int64_t num_experts, int64_t n_size,
                         int block_m, int block_n, int32_t* work_expert, int32_t* work_tile_m,
                         int32_t* work_tile_n, int64_t num_work, void* stream) {
  mgg::clear_error();
  if (num_experts < 0 || num_experts > mgg::kMaxLdsExpertsQueue)
    return set_error(MGG_ERR_UNSUPPORTED, "num_experts must be in [0, 8192]");
  if (block_m <= 0 || block_n <= 0) return set_error(MGG_ERR_INVALID, "block sizes must be > 0");
  if (n_size < 0) return set_error(MGG_ERR_INVALID, "n_size must be >= 0");
  if (num_work < 0 || num_work >= (int64_t)1 << 31)
    return set_error(MGG_ERR_INVALID, "num_work must be in [0, 2^31)");
  if (num_work > 0 && (expert_offsets == nullptr || work_expert == nullptr ||
                       work_tile_m == nullptr || work_tile_n == nullptr))
    return set_error(MGG_ERR_INVALID, "null pointer with num_work > 0");
  if (num_work > 0 && num_experts == 0)
    return set_error(MGG_ERR_INVALID, "num_work > 0 with no experts");
  return mgg::launch_build_work_queue(expert_offsets, (int32_t)num_experts, n_size, block_m,
                                      block_n, work_expert, work_tile_m, work_tile_n,
                                      (int32_t)num_work, static_cast<hipStream_t>(stream));
}

int mgg_expert_offsets_from_counts_host(const void* counts, int counts_type, int64_t num_experts,
                                        void* offsets, int out_type) {
  mgg::clear_error();
  if (num_experts < 0) return set_error(MGG_ERR_INVALID, "num_experts must be >= 0");
  if (offsets == nullptr) return set_error(MGG_ERR_INVALID, "offsets is null");
  if (num_experts > 0 && counts == nullptr) return set_error(MGG_ERR_INVALID, "counts is null");
  if ((counts_type != MGG_INT32 && counts_type != MGG_INT64) ||
      (out_type != MGG_INT32 && out_type != MGG_INT64))
    return set_error(MGG_ERR_INVALID, "counts_type and out_type must be MGG_INT32 or MGG_INT64");
  // Same arithmetic as offsets_kernel: narrow each count to int32, sum in
  // 64-bit two's complement, narrow the prefix to the output type.
  uint64_t run = 0;
  for (int64_t e = 0; e <= num_experts; ++e) {
    if (e > 0) {
      const int32_t c = counts_type == MGG_INT32
                            ? static_cast<const int32_t*>(counts)[e - 1]
                            : (int32_t) static_cast<const int64_t*>(counts)[e - 1];
      run += (uint64_t)(int64_t)c;
    }
    if (out_type == MGG_INT32)
      static_cast<int32_t*>(offsets)[e] = (int32_t)(int64_t)run;
    else
      static_cast<int64_t*>(offsets)[e] = (int64_t)run;
  }
  return MGG_OK;
}

int mgg_build_work_queue_host(const int64_t* expert_offsets, int64_t num_experts, int64_t n_size,
                              int block_m, int block_n, int32_t* work_expert,
                              int32_t* work_tile_m, int32_t* work_tile_n, int64_t num_work) {
  mgg::clear_error();
  if (num_experts < 0) return set_error(MGG_ERR_INVALID, "num_experts must be >= 0");
  if (block_m <= 0 || block_n <= 0) return set_error(MGG_ERR_INVALID, "block sizes must be > 0");
  if (n_size < 0) return set_error(MGG_ERR_INVALID, "n_size must be >= 0");
  if (num_work < 0) return set_error(MGG_ERR_INVALID, "num_work must be >= 0");
  if (num_work > 0 && (expert_offsets == nullptr || work_expert == nullptr ||
                       work_tile_m == nullptr || work_tile_n == nullptr))
    return set_error(MGG_ERR_INVALID, "null pointer with num_work > 0");
  const int64_t n_tiles = (n_size + block_n - 1) / block_n;
  int64_t w = 0;
  for (int64_t e = 0; e < num_experts; ++e) {
    const int64_t cnt = expert_offsets[e + 1] - expert_offsets[e];
    const int64_t tm_count = cnt > 0 ? (cnt + block_m - 1) / block_m : 0;
    for (int64_t tm = 0; tm < tm_count; ++tm) {
      for (int64_t tn = 0; tn < n_tiles; ++tn, ++w) {
        if (w >= num_work) return set_error(MGG_ERR_INVALID, "num_work smaller than the queue");
        work_expert[w] = (int32_t)e;
        work_tile_m[w] = (int32_t)tm;
        work_tile_n[w] = (int32_t)tn;
      }
    }
  }
  if (w != num_work) return set_error(MGG_ERR_INVALID, "num_work larger than the queue");
  return MGG_OK;
}

}  // extern "C"

namespace mgg {
namespace {

// Validation and launch shared by mgg_grouped_gemm and mgg_grouped_gemm_ex.
int grouped_gemm_impl(int dtype, int epilogue, const void* a, const void* b, void* c,
                      const int32_t* expert_offsets, int64_t m_size, int64_t k_size,
                      int64_t n_size, int64_t num_experts, int64_t lda, int64_t ldb_e,
                      int64_t ldb_k, int64_t ldc, const int32_t* work_expert,
                      const int32_t* work_tile_m, const int32_t* work_tile_n, int64_t num_work,
                      const float* a_scale, const float* b_scale, int block_m, int block_n,
                      int num_workers, int use_atomic_queue, int32_t* work_counter,
                      int report_block_m, int report_block_n, hipStream_t st,
                      const int32_t* a_rows = nullptr, int64_t a_src_rows = 0) {
  const bool fp8 = dtype == MGG_DTYPE_FP8_E4M3;
  const int base = dtype & ~MGG_B_KMAJOR;
  const bool kmajor = (dtype & MGG_B_KMAJOR) != 0;  // 16-bit B stored [E, N, K]
  if (!fp8 && ((base != MGG_DTYPE_BF16 && base != MGG_DTYPE_FP16) || (dtype & ~(MGG_B_KMAJOR | 1)) != 0))
    return set_error(MGG_ERR_UNSUPPORTED,
                     "dtype must be MGG_DTYPE_BF16 or MGG_DTYPE_FP16 (optionally | MGG_B_KMAJOR)");
  const bool b_rows_k = fp8 || kmajor;  // B's rows run along K (N rows of K values)
  if (fp8 && epilogue != MGG_EPI_NONE)
    return set_error(MGG_ERR_UNSUPPORTED, "fp8 takes no fused epilogue");
  if (fp8 && !((block_n == 128 && (block_m == 256 || block_m == 192 || block_m == 128)) ||
              (block_m == 256 && block_n == 256)))
    return set_error(MGG_ERR_UNSUPPORTED, "fp8 tiles are 256x256, 256x128, 192x128 and 128x128");
  if (epilogue != MGG_EPI_NONE && epilogue != MGG_EPI_GELU && epilogue != MGG_EPI_SWIGLU)
    return set_error(MGG_ERR_INVALID, "epilogue must be MGG_EPI_NONE, MGG_EPI_GELU or MGG_EPI_SWIGLU");
  const bool block_ok = ((block_m == 64 || block_m == 128 || block_m == 256) &&
                         (block_n == 64 || block_n == 128 || block_n == 256)) ||
                        (block_m == 128 && block_n == 512);
  if (!fp8 && !block_ok)  // fp8 tiles were checked above
    return set_error(MGG_ERR_UNSUPPORTED, "block_m/block_n must each be one of 64, 128, 256, or be 128 x 512");
  if (!epilogue_supported(epilogue, block_m, block_n))
    return set_error(MGG_ERR_UNSUPPORTED, "fused epilogues need block_m == block_n in {128, 256}");
  if (m_size < 0 || k_size < 0 || n_size < 0 || num_experts < 0)
    return set_error(MGG_ERR_INVALID, "sizes must be >= 0");
  if (m_size == 0 || n_size == 0) return MGG_OK;  // C has no elements
  // Any N: B's and C's rows need not be 16-byte aligned (16-byte DMAs and
  // stores run at any 2-byte alignment); the last chunk of a row is read as
  // it lies and stored by pairs and, for odd N, one 2-byte store.  (With N
  // odd the dword holding B's last element straddles the end of B's view;
  // the kernel adds that element's term separately.)  Odd N runs on kernel
  // instances of its own, compiled for fewer tiles.
  const bool odd_n = (n_size & 1) != 0;
  if (odd_n && !((block_m == 256 && block_n == 256) || (block_m == 128 && block_n == 128) ||
                 (block_m == 128 && block_n == 512 && !b_rows_k && epilogue == MGG_EPI_NONE)))
    return set_error(MGG_ERR_UNSUPPORTED,
                     "odd N runs on 256x256 and 128x128 tiles (and 128x512 for N-major 16-bit B "
                     "without a fused epilogue)");
  // K not a multiple of 8 (16-bit N-major B only): A is read to the next
  // multiple of 8 (those columns meet B rows that read as zeros), B's rows
  // stop at K.
  if (k_size % 8 != 0 && (fp8 || b_rows_k))
    return set_error(MGG_ERR_UNSUPPORTED, "K must be a multiple of 8 (K-major B, fp8)");
  const int64_t k_a = (k_size + 7) / 8 * 8;
  // K == 0: nothing is read (every DMA is past its descriptor, so the tiles
  // hold zeros); A's and B's strides are then unused.
  if (k_size == 0) {
    lda = 0;
    ldb_k = b_rows_k ? 0 : n_size;
    ldb_e = 0;
  }
  if (fp8 && (k_size % 16 != 0 || lda % 16 != 0 || ldb_k % 16 != 0 || ldb_e % 16 != 0))
    return set_error(MGG_ERR_UNSUPPORTED, "fp8: K and the A/B strides must be multiples of 16");
  if (epilogue == MGG_EPI_SWIGLU && n_size % 64 != 0)
    return set_error(MGG_ERR_UNSUPPORTED, "SwiGLU needs N (gate and up columns) a multiple of 64");
  const int64_t c_cols = epilogue == MGG_EPI_SWIGLU ? n_size / 2 : n_size;
  // ldb_k: stride between B's rows (K rows of N values; for fp8 and K-major
  // B, N rows of K values).
  if (report_block_m <= 0) report_block_m = block_m;
  if (report_block_n <= 0) report_block_n = block_n;
  if (lda < k_a || ldb_k < (b_rows_k ? k_size : n_size) || ldc < c_cols || ldb_e < 0)
    return set_error(MGG_ERR_INVALID, "leading dimensions smaller than the matrix extents");
  if (lda % 8 != 0 || (b_rows_k && ldb_k % 8 != 0))
    return set_error(MGG_ERR_UNSUPPORTED,
                     "lda (and ldb_k of K-major B) must be a multiple of 8 elements");
  // A and B may be null only when nothing reads them (no experts or K == 0).
  const bool reads_ab = num_experts > 0 && k_size > 0;
  if (c == nullptr || expert_offsets == nullptr || (reads_ab && (a == nullptr || b == nullptr)))
    return set_error(MGG_ERR_INVALID, "null operand pointer");
  if (fp8 && num_experts > 0 && (a_scale == nullptr || b_scale == nullptr))
    return set_error(MGG_ERR_INVALID, "fp8 needs a_scale and b_scale");
  if (!aligned16(a) || !aligned16(b) || !aligned16(c))
    return set_error(MGG_ERR_UNSUPPORTED, "operand base pointers must be 16-byte aligned");
  // In-tile byte offsets are 32-bit: BM rows of A, K+8 rows of B.
  const int64_t lim = ((int64_t)1 << 31) - 4096;
  const int64_t es = fp8 ? 1 : 2;
  const int64_t b_span = b_rows_k ? ((int64_t)block_n * ldb_k + k_size) : (k_size + 8) * ldb_k;
  if ((int64_t)block_m * lda * es + k_a * es >= lim || b_span * es >= lim)
    return set_error(MGG_ERR_UNSUPPORTED, "row strides too large for 32-bit tile offsets");
  // Gathered A: the A-block tile (256x256, 16-bit A, N-major B) with the
  // device-derived queue; offsets into the source matrix are 32-bit.
  if (a_rows != nullptr) {
    if (fp8 || kmajor || block_m != 256 || block_n != 256 || num_work >= 0)
      return set_error(MGG_ERR_UNSUPPORTED,
                       "gathered A needs 16-bit N-major B, 256x256 tiles and the device-derived queue");
    if (a_src_rows < 0) return set_error(MGG_ERR_INVALID, "a_src_rows must be >= 0");
    if (a_src_rows * lda * es + k_a * es >= lim)
      return set_error(MGG_ERR_UNSUPPORTED, "gathered A source too large for 32-bit offsets");
  }

  int workers = num_workers;
  if (workers <= 0) {
    int device = 0;
    hipError_t err = hipGetDevice(&device);
    if (err != hipSuccess) return hip_error(err, "hipGetDevice");
    err = hipDeviceGetAttribute(&workers, hipDeviceAttributeMultiprocessorCount, device);
    if (err != hipSuccess) return hip_error(err, "hipDeviceGetAttribute");
  }
  if (workers > 65536) return set_error(MGG_ERR_INVALID, "num_workers must be <= 65536");

  const int64_t n_tiles = (n_size + block_n - 1) / block_n;
  if (num_work >= 0) {
    if (num_work > 0 && (work_expert == nullptr || work_tile_m == nullptr || work_tile_n == nullptr))
      return set_error(MGG_ERR_INVALID, "null work queue with num_work > 0");
    if (num_work + workers >= ((int64_t)1 << 31))
      return set_error(MGG_ERR_INVALID, "num_work + num_workers must be < 2^31");
  } else {
    if (num_experts > kMaxLdsExpertsGemm)
      return set_error(MGG_ERR_UNSUPPORTED,
                       "the device-derived queue supports at most 2048 experts; pass a "
                       "prebuilt queue");
    // Upper bound of the queue length for offsets inside [0, M].
    const int64_t bound = (m_size / block_m + num_experts + 1) * n_tiles;
    if (bound + workers >= ((int64_t)1 << 31))
      return set_error(MGG_ERR_INVALID, "queue length may exceed 2^31");
  }

  GemmParams p{};
  p.a = static_cast<const uint16_t*>(a);
  p.b = static_cast<const uint16_t*>(b);
  p.c = static_cast<uint16_t*>(c);
  p.offsets = expert_offsets;
  p.q_expert = num_work >= 0 ? work_expert : nullptr;
  p.q_tile_m = num_work >= 0 ? work_tile_m : nullptr;
  p.q_tile_n = num_work >= 0 ? work_tile_n : nullptr;
  p.m = m_size;
  p.k = k_size;
  p.n = n_size;
  p.lda = lda;
  p.ldb_e = ldb_e;
  p.ldb_k = ldb_k;
  p.ldc = ldc;
  p.a_scale = a_scale;
  p.b_scale = b_scale;
  p.num_experts = (int32_t)num_experts;
  p.num_work = num_work >= 0 ? (int32_t)num_work : -1;
  p.atomic = use_atomic_queue ? 1 : 0;
  p.remap_xcd = 1;
  p.report_bm = report_block_m;
  p.report_bn = report_block_n;
  p.clock_probe = clock_probe();
  p.a_rows = a_rows;
  p.a_src_rows = a_rows != nullptr ? a_src_rows : 0;
  if (p.atomic) {
    int rc = counter_for(st, &p.counter, &p.epoch, &p.next_epoch);
    if (rc != MGG_OK) return rc;
    p.report = work_counter;
    if (num_work < 0 && k_size > 0) {
      rc = split_space_for(st, block_m, block_n, &p);
      if (rc != MGG_OK) return rc;
    }
  }
  return odd_n ? launch_grouped_gemm_odd(dtype, epilogue, block_m, block_n, p, workers, st)
               : launch_grouped_gemm(dtype, epilogue, block_m, block_n, p, workers, st);
}

}  // namespace
}  // namespace mgg

extern "C" {

int mgg_grouped_gemm(int dtype, const void* a, const void* b, void* c,
                     const int32_t* expert_offsets, int64_t m_size, int64_t k_size, int64_t n_size,
                     int64_t num_experts, int64_t lda, int64_t ldb_e, int64_t ldb_k, int64_t ldc,
                     const int32_t* work_expert, const int32_t* work_tile_m,
                     const int32_t* work_tile_n, int64_t num_work, int block_m, int block_n,
                     int num_workers, int use_atomic_queue, int32_t* work_counter,
                     int report_block_m, int report_block_n, void* stream) {
  mgg::clear_error();
  return mgg::grouped_gemm_impl(dtype, MGG_EPI_NONE, a, b, c, expert_offsets, m_size, k_size,
                                n_size, num_experts, lda, ldb_e, ldb_k, ldc, work_expert,
                                work_tile_m, work_tile_n, num_work, nullptr, nullptr, block_m,
                                block_n, num_workers, use_atomic_queue, work_counter,
                                report_block_m, report_block_n, static_cast<hipStream_t>(stream));
}

int mgg_grouped_gemm_ex(int dtype, int epilogue, const void* a, const void* b, void* c,
                        const int32_t* expert_offsets, int64_t m_size, int64_t k_size,
                        int64_t n_size, int64_t num_experts, int64_t lda, int64_t ldb_e,
                        int64_t ldb_k, int64_t ldc, const int32_t* work_expert,
                        const int32_t* work_tile_m, const int32_t* work_tile_n, int64_t num_work,
                        int block_m, int block_n, int num_workers, int use_atomic_queue,
                        int32_t* work_counter, int report_block_m, int report_block_n,
                        void* stream) {
  mgg::clear_error();
  if (dtype == MGG_DTYPE_FP8_E4M3)
    return set_error(MGG_ERR_UNSUPPORTED, "fp8 goes through mgg_grouped_gemm_fp8");
  return mgg::grouped_gemm_impl(dtype, epilogue, a, b, c, expert_offsets, m_size, k_size, n_size,
                                num_experts, lda, ldb_e, ldb_k, ldc, work_expert, work_tile_m,
                                work_tile_n, num_work, nullptr, nullptr, block_m, block_n,
                                num_workers, use_atomic_queue, work_counter, report_block_m,
                                report_block_n, static_cast<hipStream_t>(stream));
}

int mgg_grouped_gemm_gathered(int dtype, int epilogue, const void* a, const int32_t* a_rows,
                              int64_t a_src_rows, const void* b, void* c,
                              const int32_t* expert_offsets, int64_t m_size, int64_t k_size,
                              int64_t n_size, int64_t num_experts, int64_t lda, int64_t ldb_e,
                              int64_t ldb_k, int64_t ldc, int num_workers, int use_atomic_queue,
                              void* stream) {
  mgg::clear_error();
  if (a_rows == nullptr && m_size > 0 && n_size > 0 && num_experts > 0 && k_size > 0)
    return set_error(MGG_ERR_INVALID, "null a_rows");
  if (dtype == MGG_DTYPE_FP8_E4M3)
    return set_error(MGG_ERR_UNSUPPORTED, "gathered A takes 16-bit operands");
  return mgg::grouped_gemm_impl(dtype, epilogue, a, b, c, expert_offsets, m_size, k_size, n_size,
                                num_experts, lda, ldb_e, ldb_k, ldc, nullptr, nullptr, nullptr, -1,
                                nullptr, nullptr, 256, 256, num_workers, use_atomic_queue, nullptr,
                                256, 256, static_cast<hipStream_t>(stream), a_rows, a_src_rows);
}

int mgg_grouped_gemm_fp8(const void* a, const void* b, void* c, const int32_t* expert_offsets,
                         const float* a_scale, const float* b_scale, int64_t m_size,
                         int64_t k_size, int64_t n_size, int64_t num_experts, int64_t lda,
                         int64_t ldb_e, int64_t ldb_n, int64_t ldc, const int32_t* work_expert,
                         const int32_t* work_tile_m, const int32_t* work_tile_n,
                         int64_t num_work, int block_m, int block_n, int num_workers,
                         int use_atomic_queue, int32_t* work_counter, int report_block_m,
                         int report_block_n, void* stream) {
  mgg::clear_error();
  return mgg::grouped_gemm_impl(MGG_DTYPE_FP8_E4M3, MGG_EPI_NONE, a, b, c, expert_offsets, m_size,
                                k_size, n_size, num_experts, lda, ldb_e, ldb_n, ldc, work_expert,
                                work_tile_m, work_tile_n, num_work, a_scale, b_scale, block_m,
                                block_n, num_workers, use_atomic_queue, work_counter,
                                report_block_m, report_block_n, static_cast<hipStream_t>(stream));
}

int mgg_debug_set_dequeue_counter(uint64_t value, void* stream) {
  mgg::clear_error();
  unsigned long long* word = nullptr;
  const hipStream_t st = static_cast<hipStream_t>(stream);
  uint32_t unused_epoch = 0, unused_next = 0;
  const int rc = mgg::counter_for(st, &word, &unused_epoch, &unused_next, false);
  if (rc != MGG_OK) return rc;
  return mgg::launch_fill_u64(word, 1, (unsigned long long)value, st);
}

int mgg_debug_set_split_flags(uint64_t value, void* stream) {
  mgg::clear_error();
  const hipStream_t st = static_cast<hipStream_t>(stream);
  const mgg::SplitSpace* sp = nullptr;
  const int rc = mgg::split_space(st, false, &sp);
  if (rc != MGG_OK) return rc;
  if (sp == nullptr) return set_error(MGG_ERR_INVALID, "no split workspace on this stream yet");
  return mgg::launch_fill_u64(sp->flags, (int)sp->flag_words, (unsigned long long)value, st);
}

int mgg_debug_counter_slots(int device, int* held) {
  mgg::clear_error();
  if (held == nullptr) return set_error(MGG_ERR_INVALID, "held is null");
  std::lock_guard<std::mutex> lock(mgg::g_slots.mu);
  *held = 0;
  if (device >= 0 && device < (int)mgg::g_slots.used.size())
    *held = mgg::g_slots.used[device] - (int)mgg::g_slots.freed[device].size();
  return MGG_OK;
}

int mgg_reserve_split_workspace(void* stream) {
  mgg::clear_error();
  const hipStream_t st = static_cast<hipStream_t>(stream);
  if (st != nullptr) {  // (allocating, and clearing the flags, under capture would be recorded)
    hipStreamCaptureStatus capture = hipStreamCaptureStatusNone;
    const hipError_t err = hipStreamIsCapturing(st, &capture);
    if (err != hipSuccess) return mgg::hip_error(err, "hipStreamIsCapturing");
    if (capture != hipStreamCaptureStatusNone)
      return set_error(MGG_ERR_INVALID, "the split workspace cannot be reserved under graph capture");
  }
  const mgg::SplitSpace* sp = nullptr;
  return mgg::split_space(st, true, &sp);
}

int mgg_split_workspace_bytes(void* stream, int64_t* bytes) {
  mgg::clear_error();
  if (bytes == nullptr) return set_error(MGG_ERR_INVALID, "bytes is null");
  const mgg::SplitSpace* sp = nullptr;
  const int rc = mgg::split_space(static_cast<hipStream_t>(stream), false, &sp);
  if (rc != MGG_OK) return rc;
  *bytes = sp != nullptr ? sp->bytes + sp->flag_words * 8 : 0;
  return MGG_OK;
}

int mgg_set_split_last_round(int enabled) {
  mgg::clear_error();
  mgg::g_split_enabled.store(enabled ? 1 : 0);
  return MGG_OK;
}

int64_t mgg_dispatch_layout_workspace_bytes(int64_t num_tokens, int top_k, int64_t num_experts) {
  if (num_tokens < 0 || top_k < 0 || num_experts < 0) return -1;
  return mgg::layout_chunks(num_tokens * top_k) * num_experts * (int64_t)sizeof(int32_t);
}

int mgg_dispatch_layout(const void* topk_idx, int idx_type, int64_t num_tokens, int top_k,
                        int64_t num_experts, int32_t* counts, int32_t* offsets,
                        int32_t* slot_position, int32_t* token_index, int32_t* row_assignment,
                        void* workspace, int64_t workspace_bytes, void* stream) {
  mgg::clear_error();
  if (idx_type != MGG_INT32 && idx_type != MGG_INT64)
    return set_error(MGG_ERR_INVALID, "idx_type must be MGG_INT32 or MGG_INT64");
  if (num_tokens < 0 || top_k < 0 || num_experts < 0)
    return set_error(MGG_ERR_INVALID, "sizes must be >= 0");
  if (num_experts > mgg::kMaxLayoutExperts)
    return set_error(MGG_ERR_UNSUPPORTED, "the dispatch layout supports at most 8192 experts");
  const int64_t A = num_tokens * top_k;
  if (A >= ((int64_t)1 << 31)) return set_error(MGG_ERR_UNSUPPORTED, "num_tokens * top_k must be < 2^31");
  if (workspace_bytes < mgg_dispatch_layout_workspace_bytes(num_tokens, top_k, num_experts))
    return set_error(MGG_ERR_INVALID, "workspace smaller than mgg_dispatch_layout_workspace_bytes");
  if (offsets == nullptr || (num_experts > 0 && counts == nullptr))
    return set_error(MGG_ERR_INVALID, "null counts/offsets");
  if (A > 0 && (topk_idx == nullptr || slot_position == nullptr || token_index == nullptr ||
                row_assignment == nullptr || (num_experts > 0 && workspace == nullptr)))
    return set_error(MGG_ERR_INVALID, "null index or output pointer");
  return mgg::launch_dispatch_layout(topk_idx, idx_type, num_tokens, top_k, (int32_t)num_experts,
                                     counts, offsets, slot_position, token_index, row_assignment,
                                     static_cast<int32_t*>(workspace),
                                     static_cast<hipStream_t>(stream));
}

int mgg_debug_set_clock_probe(uint64_t* probe) {
  mgg::clear_error();
  if (probe != nullptr && (reinterpret_cast<uintptr_t>(probe) & 7u) != 0)
    return set_error(MGG_ERR_INVALID, "probe must be 8-byte aligned");
  mgg::g_clock_probe.store(reinterpret_cast<unsigned long long*>(probe));
  return MGG_OK;
}

int mgg_dispatch_layout_noalloc(const void* topk_idx, int idx_type, int64_t num_tokens, int top_k,
                                int64_t num_experts, int32_t* counts, int32_t* offsets,
                                int32_t* slot_position, int32_t* token_index,
                                int32_t* row_assignment, void* stream) {
  mgg::clear_error();
  const int64_t need = mgg_dispatch_layout_workspace_bytes(num_tokens, top_k, num_experts);
  if (need < 0) return set_error(MGG_ERR_INVALID, "sizes must be >= 0");
  if (need > mgg::kScratchBytes)
    return set_error(MGG_ERR_UNSUPPORTED,
                     "mgg_dispatch_layout_noalloc: the layout needs " + std::to_string(need) +
                         " bytes of workspace (ceil(T*top_k/1024) * E * 4), more than its "
                         "1 MiB scratch; pass a workspace to mgg_dispatch_layout");
  int32_t* ws = nullptr;
  const int rc = mgg::scratch_for_current_device(&ws);
  if (rc != MGG_OK) return rc;
  return mgg_dispatch_layout(topk_idx, idx_type, num_tokens, top_k, num_experts, counts, offsets,
                             slot_position, token_index, row_assignment, ws, need, stream);
}

int mgg_gather_rows(int dtype, const void* x, int64_t ld_x, const int32_t* token_index,
                    const int32_t* num_rows, int64_t max_rows, int64_t hidden, void* out,
                    int64_t ld_out, void* stream) {
  mgg::clear_error();
  if (dtype != MGG_DTYPE_BF16 && dtype != MGG_DTYPE_FP16)
    return set_error(MGG_ERR_UNSUPPORTED, "dtype must be MGG_DTYPE_BF16 or MGG_DTYPE_FP16");
  if (max_rows < 0 || hidden < 0) return set_error(MGG_ERR_INVALID, "sizes must be >= 0");
  if (max_rows == 0 || hidden == 0) return MGG_OK;
  if (ld_x < hidden || ld_out < hidden)
    return set_error(MGG_ERR_INVALID, "leading dimensions smaller than the row length");
  if (x == nullptr || token_index == nullptr || out == nullptr)
    return set_error(MGG_ERR_INVALID, "null pointer");
  return mgg::launch_gather_rows(x, ld_x, token_index, num_rows, max_rows, hidden, 2, out, ld_out,
                                 static_cast<hipStream_t>(stream));
}

int mgg_combine_rows(int dtype, const void* y, int64_t ld_y, const int32_t* slot_position,
                     const float* weights, int64_t num_tokens, int top_k, int64_t hidden,
                     void* out, int64_t ld_out, void* stream) {
  mgg::clear_error();
  if (dtype != MGG_DTYPE_BF16 && dtype != MGG_DTYPE_FP16)
    return set_error(MGG_ERR_UNSUPPORTED, "dtype must be MGG_DTYPE_BF16 or MGG_DTYPE_FP16");
  if (num_tokens < 0 || top_k < 0 || hidden < 0)
    return set_error(MGG_ERR_INVALID, "sizes must be >= 0");
  if (num_tokens == 0 || hidden == 0) return MGG_OK;
  if (ld_out < hidden || (top_k > 0 && ld_y < hidden))
    return set_error(MGG_ERR_INVALID, "leading dimensions smaller than the row length");
  if (out == nullptr || (top_k > 0 && (y == nullptr || slot_position == nullptr || weights == nullptr)))
    return set_error(MGG_ERR_INVALID, "null pointer");
  return mgg::launch_combine_rows(dtype, y, ld_y, slot_position, weights, num_tokens, top_k,
                                  hidden, out, ld_out, static_cast<hipStream_t>(stream));
}

}  // extern "C"
