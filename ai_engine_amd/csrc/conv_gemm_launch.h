// conv_gemm_launch.h -- host-side launchers of the MFMA conv-GEMM kernels.
#pragma once

#include <hip/hip_runtime.h>

#include "conv_gemm_impl.h"

namespace aih {

// Output-channel tile widths that have a kernel instantiation.
constexpr int kGemmBN[] = {32, 64, 96, 128, 160, 256};

// One instantiation table per activation dtype (separate translation units).
hipError_t launch_conv_gemm_f32(const GemmArgs &a, int dtw, int bn, bool igemm, hipStream_t st);
hipError_t launch_conv_gemm_f16(const GemmArgs &a, int dtw, int bn, bool igemm, hipStream_t st);
hipError_t launch_conv_gemm_bf16(const GemmArgs &a, int dtw, int bn, bool igemm, hipStream_t st);
hipError_t launch_splitk_reduce(const GemmArgs &a, int dta, hipStream_t st);

inline hipError_t launch_conv_gemm(const GemmArgs &a, int dta, int dtw, int bn, bool igemm, hipStream_t st) {
  switch (dta) {
    case DT_F32: return launch_conv_gemm_f32(a, dtw, bn, igemm, st);
    case DT_F16: return launch_conv_gemm_f16(a, dtw, bn, igemm, st);
    case DT_BF16: return launch_conv_gemm_bf16(a, dtw, bn, igemm, st);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace aih
