// conv_gemm_f32.hip -- conv-GEMM instantiations for fp32 activations
// (weights fp32, f16 or bf16; fp32 MFMA) and the split-K reduction.
#include "conv_gemm_launch.h"

namespace aih {

template <int DTW>
static hipError_t launch_w(const GemmArgs &a, int bn, bool igemm, hipStream_t st) {
  if (igemm) {
    AIH_GEMM_BN_SWITCH(DT_F32, DTW, true, false, bn, a, st)
  } else {
    AIH_GEMM_BN_SWITCH(DT_F32, DTW, false, false, bn, a, st)
  }
}

hipError_t launch_conv_gemm_f32(const GemmArgs &a, int dtw, int bn, bool igemm, hipStream_t st) {
  switch (dtw) {
    case DT_F32: return launch_w<DT_F32>(a, bn, igemm, st);
    case DT_F16: return launch_w<DT_F16>(a, bn, igemm, st);
    case DT_BF16: return launch_w<DT_BF16>(a, bn, igemm, st);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_splitk_reduce(const GemmArgs &a, int dta, hipStream_t st) {
  const size_t nvec = (size_t)a.M * a.N4 / 4;
  const dim3 grid((unsigned)((nvec + 255) / 256));
  switch (dta) {
    case DT_F32:
      hipLaunchKernelGGL(splitk_reduce_kernel<DT_F32>, grid, dim3(256), 0, st, a.partial, a.nsplit, a.M, a.N4,
                         a.bias, a.res, a.y, a.act, a.has_res);
      break;
    case DT_F16:
      hipLaunchKernelGGL(splitk_reduce_kernel<DT_F16>, grid, dim3(256), 0, st, a.partial, a.nsplit, a.M, a.N4,
                         a.bias, a.res, a.y, a.act, a.has_res);
      break;
    case DT_BF16:
      hipLaunchKernelGGL(splitk_reduce_kernel<DT_BF16>, grid, dim3(256), 0, st, a.partial, a.nsplit, a.M, a.N4,
                         a.bias, a.res, a.y, a.act, a.has_res);
      break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace aih
