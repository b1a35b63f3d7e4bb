// Launches of the grouped GEMM kernel (mgg_gemm_kernel.h) for N even: the
// instances every even N runs, bf16/fp16 with N-major and K-major B, fused
// epilogues, gathered A, and fp8.  Odd N goes to mgg_gemm_odd.hip.
#include "mgg_gemm_kernel.h"

namespace mgg {
namespace {
__global__ void fill_u64_kernel(unsigned long long* ptr, int count, unsigned long long value) {
  for (int i = threadIdx.x; i < count; i += blockDim.x) ptr[i] = value;
}

template <class T, int EPI>
int launch_typed(int block_m, int block_n, const GemmParams& p, int workers, hipStream_t stream) {
#define MGG_CASE(BM_, BN_, SBK_, NS_, NW_)                                                      \
  if (block_m == BM_ && block_n == BN_) {                                                      \
    hipLaunchKernelGGL((grouped_gemm_kernel<BM_, BN_, SBK_, NS_, NW_, T, EPI>), dim3(workers), \
                       dim3(NW_ * 64), 0, stream, p);                                           \
    return MGG_OK;                                                                              \
  }
  // (tile, K per stage, LDS stages, waves): 64-wide K stages (128-byte A
  // rows) and as many stages as the LDS budget holds, except the 256x256
  // tile (see MGG_SBK256).  Fused epilogues are compiled for the 256x256 and
  // 128x128 tiles (two 32-column blocks per wave).
  constexpr int kSbk256 = T::kBKMajor ? MGG_KM_SBK256 : MGG_SBK256;
  constexpr int kNs256 = T::kBKMajor ? MGG_KM_NS256 : MGG_NS256;
  MGG_CASE(256, 256, kSbk256, kNs256, MGG_NW256)
  MGG_CASE(128, 128, 64, 4, 4)
  if constexpr (EPI == kEpiNone) {
    MGG_CASE(256, 128, 64, 3, 4)
    MGG_CASE(128, 256, 64, 3, 4)
    MGG_CASE(128, 64, 64, 4, 4)
    MGG_CASE(64, 128, 64, 4, 4)
    MGG_CASE(64, 64, 64, 4, 4)
    MGG_CASE(256, 64, 64, 3, 4)
    MGG_CASE(64, 256, 64, 3, 4)
    MGG_CASE(128, 512, 32, 3, 8)
  }
#undef MGG_CASE
  return set_error(MGG_ERR_UNSUPPORTED, EPI == kEpiNone
                                            ? "block_m/block_n must each be one of 64, 128, 256"
                                            : "fused epilogues need block_m == block_n in {128, 256}");
}

// fp8: 128-byte rows of K (K-wide 128 stages, two 64-deep MFMA steps), eight
// waves (two per SIMD) on 256x256, 256x128, 192x128 and 128x128 tiles.  The
// 256x256 tile makes the fewest L2 requests per FLOP; it fits the 256
// registers a wave has at two waves per SIMD only with its A fragments
// single-buffered (kASingle).  The narrower tiles suit experts of up to 256
// rows, where a 256x256 tile would be mostly padding.
int launch_fp8(int block_m, int block_n, const GemmParams& p, int workers, hipStream_t stream) {
#define MGG_CASE(BM_, BN_, SBK_, NS_, NW_)                                                    \
  if (block_m == BM_ && block_n == BN_) {                                                    \
    hipLaunchKernelGGL((grouped_gemm_kernel<BM_, BN_, SBK_, NS_, NW_, Fp8, kEpiNone>),       \
                       dim3(workers), dim3(NW_ * 64), 0, stream, p);                          \
    return MGG_OK;                                                                            \
  }
  MGG_CASE(256, 256, 128, 2, MGG_FP8_NW)
  MGG_CASE(256, 128, 128, 3, MGG_FP8_NW)
  MGG_CASE(192, 128, 128, 3, MGG_FP8_NW)
  MGG_CASE(128, 128, 128, 4, MGG_FP8_NW)
#undef MGG_CASE
  return set_error(MGG_ERR_UNSUPPORTED, "fp8 tiles are 256x256, 256x128, 192x128 and 128x128");
}

// Gathered A: the 256x256 A-block tile only (the host checks the shape).
template <class T, int EPI>
int launch_gathered(const GemmParams& p, int workers, hipStream_t stream) {
  hipLaunchKernelGGL((grouped_gemm_kernel<256, 256, MGG_SBK256, MGG_NS256, MGG_NW256, T, EPI | kEpiGather>),
                     dim3(workers), dim3(MGG_NW256 * 64), 0, stream, p);
  return MGG_OK;
}

template <class T>
int launch_epi(int epilogue, int block_m, int block_n, const GemmParams& p, int workers,
               hipStream_t stream) {
  if constexpr (!T::kBKMajor && !T::kScaled) {
    if (p.a_rows != nullptr) {
      if (block_m != 256 || block_n != 256)
        return set_error(MGG_ERR_UNSUPPORTED, "gathered A needs 256x256 tiles");
      switch (epilogue) {
        case kEpiNone: return launch_gathered<T, kEpiNone>(p, workers, stream);
        case kEpiGelu: return launch_gathered<T, kEpiGelu>(p, workers, stream);
        case kEpiSwiglu: return launch_gathered<T, kEpiSwiglu>(p, workers, stream);
        default: return set_error(MGG_ERR_INVALID, "unknown epilogue");
      }
    }
  } else {
    if (p.a_rows != nullptr) return set_error(MGG_ERR_UNSUPPORTED, "gathered A needs N-major 16-bit B");
  }
  switch (epilogue) {
    case kEpiNone: return launch_typed<T, kEpiNone>(block_m, block_n, p, workers, stream);
    case kEpiGelu: return launch_typed<T, kEpiGelu>(block_m, block_n, p, workers, stream);
    case kEpiSwiglu: return launch_typed<T, kEpiSwiglu>(block_m, block_n, p, workers, stream);
    default: return set_error(MGG_ERR_INVALID, "unknown epilogue");
  }
}

}  // namespace

bool epilogue_supported(int epilogue, int block_m, int block_n) {
  if (epilogue == kEpiNone) return true;
  return block_m == block_n && (block_m == 128 || block_m == 256);
}

int launch_grouped_gemm(int dtype, int epilogue, int block_m, int block_n, const GemmParams& p,
                        int workers, hipStream_t stream) {
  int rc;
  if (dtype == MGG_DTYPE_BF16)
    rc = launch_epi<Bf16>(epilogue, block_m, block_n, p, workers, stream);
  else if (dtype == MGG_DTYPE_FP16)
    rc = launch_epi<F16>(epilogue, block_m, block_n, p, workers, stream);
  else if (dtype == (MGG_DTYPE_BF16 | MGG_B_KMAJOR))
    rc = launch_epi<Bf16K>(epilogue, block_m, block_n, p, workers, stream);
  else if (dtype == (MGG_DTYPE_FP16 | MGG_B_KMAJOR))
    rc = launch_epi<F16K>(epilogue, block_m, block_n, p, workers, stream);
  else if (dtype == MGG_DTYPE_FP8_E4M3 && epilogue == kEpiNone)
    rc = launch_fp8(block_m, block_n, p, workers, stream);
  else
    return set_error(MGG_ERR_UNSUPPORTED, "unsupported dtype / epilogue combination");
  if (rc != MGG_OK) return rc;
  return hip_error(hipGetLastError(), "grouped_gemm_kernel launch");
}

int launch_fill_u64(unsigned long long* ptr, int count, unsigned long long value, hipStream_t stream) {
  hipLaunchKernelGGL(fill_u64_kernel, dim3(1), dim3(64), 0, stream, ptr, count, value);
  return hip_error(hipGetLastError(), "fill_u64_kernel launch");
}

}  // namespace mgg
