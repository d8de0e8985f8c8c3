// conv_gemm_f16.hip -- conv-GEMM kernel instantiations for f16 activations.
#include "conv_gemm_launch.h"

namespace aih {

template <int DTW, int BN>
static hipError_t launch_bn(const GemmArgs &a, bool igemm, hipStream_t st) {
  const dim3 grid(a.mtiles * a.ntiles * a.nsplit);
  if (igemm)
    hipLaunchKernelGGL((conv_gemm_kernel<DT_F16, DTW, BN, true>), grid, dim3(GEMM_THREADS), 0, st, a);
  else
    hipLaunchKernelGGL((conv_gemm_kernel<DT_F16, DTW, BN, false>), grid, dim3(GEMM_THREADS), 0, st, a);
  return hipGetLastError();
}

template <int DTW>
static hipError_t launch_w(const GemmArgs &a, int bn, bool igemm, hipStream_t st) {
  switch (bn) {
    case 32: return launch_bn<DTW, 32>(a, igemm, st);
    case 64: return launch_bn<DTW, 64>(a, igemm, st);
    case 96: return launch_bn<DTW, 96>(a, igemm, st);
    case 128: return launch_bn<DTW, 128>(a, igemm, st);
    case 160: return launch_bn<DTW, 160>(a, igemm, st);
    case 256: return launch_bn<DTW, 256>(a, igemm, st);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_conv_gemm_f16(const GemmArgs &a, int dtw, int bn, bool igemm, hipStream_t st) {
  switch (dtw) {
    case DT_F16: return launch_w<DT_F16>(a, bn, igemm, st);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace aih
