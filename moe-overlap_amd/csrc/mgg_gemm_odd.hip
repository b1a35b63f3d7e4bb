// Launches of the grouped GEMM kernel (mgg_gemm_kernel.h) for odd N: the
// kEpiOddN instances, which end C's rows in a 2-byte store and, with N-major
// 16-bit B, add the term of B's last element themselves.  Compiled for the
// tiles the drop-in computes with (256x256, 128x128; 128x512 for N-major
// 16-bit B without a fused epilogue); the host rejects others for odd N.
#include "mgg_gemm_kernel.h"

namespace mgg {
namespace {

template <int BM, int BN, int SBK, int NS, int NW, class T, int EPI>
int launch_one(const GemmParams& p, int workers, hipStream_t stream) {
  hipLaunchKernelGGL((grouped_gemm_kernel<BM, BN, SBK, NS, NW, T, EPI | kEpiOddN>), dim3(workers),
                     dim3(NW * 64), 0, stream, p);
  return MGG_OK;
}

// The same (tile, K per stage, LDS stages, waves) as the even-N instances.
template <class T, int EPI>
int launch_typed_odd(int block_m, int block_n, const GemmParams& p, int workers,
                     hipStream_t stream) {
  constexpr int kSbk256 = T::kBKMajor ? MGG_KM_SBK256 : MGG_SBK256;
  constexpr int kNs256 = T::kBKMajor ? MGG_KM_NS256 : MGG_NS256;
  if (block_m == 256 && block_n == 256)
    return launch_one<256, 256, kSbk256, kNs256, MGG_NW256, T, EPI>(p, workers, stream);
  if (block_m == 128 && block_n == 128)
    return launch_one<128, 128, 64, 4, 4, T, EPI>(p, workers, stream);
  if constexpr (EPI == kEpiNone && !T::kBKMajor) {
    if (block_m == 128 && block_n == 512)
      return launch_one<128, 512, 32, 3, 8, T, EPI>(p, workers, stream);
  }
  return set_error(MGG_ERR_UNSUPPORTED, "no odd-N kernel for this tile");
}

int launch_fp8_odd(int block_m, int block_n, const GemmParams& p, int workers,
                   hipStream_t stream) {
  if (block_m == 256 && block_n == 256)
    return launch_one<256, 256, 128, 2, MGG_FP8_NW, Fp8, kEpiNone>(p, workers, stream);
  if (block_m == 128 && block_n == 128)
    return launch_one<128, 128, 128, 4, MGG_FP8_NW, Fp8, kEpiNone>(p, workers, stream);
  return set_error(MGG_ERR_UNSUPPORTED, "no odd-N fp8 kernel for this tile");
}

template <class T>
int launch_epi_odd(int epilogue, int block_m, int block_n, const GemmParams& p, int workers,
                   hipStream_t stream) {
  if constexpr (!T::kBKMajor) {
    if (p.a_rows != nullptr) {  // gathered A: 256x256 (the host checks the shape)
      if (epilogue == kEpiNone)
        return launch_one<256, 256, MGG_SBK256, MGG_NS256, MGG_NW256, T, kEpiNone | kEpiGather>(
            p, workers, stream);
      if (epilogue == kEpiGelu)
        return launch_one<256, 256, MGG_SBK256, MGG_NS256, MGG_NW256, T, kEpiGelu | kEpiGather>(
            p, workers, stream);
      return set_error(MGG_ERR_UNSUPPORTED, "no odd-N kernel for this epilogue");
    }
  } else {
    if (p.a_rows != nullptr) return set_error(MGG_ERR_UNSUPPORTED, "gathered A needs N-major 16-bit B");
  }
  switch (epilogue) {
    case kEpiNone: return launch_typed_odd<T, kEpiNone>(block_m, block_n, p, workers, stream);
    case kEpiGelu: return launch_typed_odd<T, kEpiGelu>(block_m, block_n, p, workers, stream);
    default: return set_error(MGG_ERR_UNSUPPORTED, "no odd-N kernel for this epilogue");
  }
}

}  // namespace

int launch_grouped_gemm_odd(int dtype, int epilogue, int block_m, int block_n, const GemmParams& p,
                            int workers, hipStream_t stream) {
  int rc;
  if (dtype == MGG_DTYPE_BF16)
    rc = launch_epi_odd<Bf16>(epilogue, block_m, block_n, p, workers, stream);
  else if (dtype == MGG_DTYPE_FP16)
    rc = launch_epi_odd<F16>(epilogue, block_m, block_n, p, workers, stream);
  else if (dtype == (MGG_DTYPE_BF16 | MGG_B_KMAJOR))
    rc = launch_epi_odd<Bf16K>(epilogue, block_m, block_n, p, workers, stream);
  else if (dtype == (MGG_DTYPE_FP16 | MGG_B_KMAJOR))
    rc = launch_epi_odd<F16K>(epilogue, block_m, block_n, p, workers, stream);
  else if (dtype == MGG_DTYPE_FP8_E4M3 && epilogue == kEpiNone)
    rc = launch_fp8_odd(block_m, block_n, p, workers, stream);
  else
    return set_error(MGG_ERR_UNSUPPORTED, "unsupported dtype / epilogue combination");
  if (rc != MGG_OK) return rc;
  return hip_error(hipGetLastError(), "grouped_gemm_kernel launch");
}

}  // namespace mgg
