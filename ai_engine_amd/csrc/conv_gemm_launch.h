// conv_gemm_launch.h -- host-side launchers of the MFMA conv-GEMM kernels.
#pragma once

#include <hip/hip_runtime.h>

#include <algorithm>

#include "conv_gemm_impl.h"

namespace aih {

// Output-channel tile widths that have a kernel instantiation.
constexpr int kGemmBN[] = {32, 64, 96, 128, 160};

// Persistent launch: as many workgroups as fit on the device at once (from
// the occupancy of this instantiation), capped by the number of tiles.
template <int DTA, int DTW, int BN, bool IG, bool PAIR>
hipError_t launch_gemm_inst(const GemmArgs &a, hipStream_t st) {
  auto kern = conv_gemm_kernel<DTA, DTW, BN, IG, PAIR>;
  static const int per_cu = [kern] {
    int nb = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, kern, GEMM_THREADS, 0) != hipSuccess || nb < 1) nb = 1;
    return nb;
  }();
  const uint32_t slots = device_cus() * (uint32_t)per_cu;
  const uint32_t grid = std::min(a.ntiles_total, slots);
  hipLaunchKernelGGL(kern, dim3(grid), dim3(GEMM_THREADS), 0, st, a);
  return hipGetLastError();
}

// One instantiation table per activation dtype (separate translation units).
hipError_t launch_conv_gemm_f32(const GemmArgs &a, int dtw, int bn, bool igemm, hipStream_t st);
hipError_t launch_conv_gemm_f16(const GemmArgs &a, int bn, bool igemm, bool pair, hipStream_t st);
hipError_t launch_conv_gemm_bf16(const GemmArgs &a, int bn, bool igemm, bool pair, hipStream_t st);
hipError_t launch_splitk_reduce(const GemmArgs &a, int dta, hipStream_t st);

inline hipError_t launch_conv_gemm(const GemmArgs &a, int dta, int dtw, int bn, bool igemm, bool pair,
                                   hipStream_t st) {
  switch (dta) {
    case DT_F32: return launch_conv_gemm_f32(a, dtw, bn, igemm, st);
    case DT_F16: return dtw == DT_F16 ? launch_conv_gemm_f16(a, bn, igemm, pair, st) : hipErrorInvalidValue;
    case DT_BF16: return dtw == DT_BF16 ? launch_conv_gemm_bf16(a, bn, igemm, pair, st) : hipErrorInvalidValue;
    default: return hipErrorInvalidValue;
  }
}

#define AIH_GEMM_BN_SWITCH(DTA, DTW, IG, PAIR, bn, a, st)                          \
  switch (bn) {                                                                    \
    case 32: return launch_gemm_inst<DTA, DTW, 32, IG, PAIR>(a, st);               \
    case 64: return launch_gemm_inst<DTA, DTW, 64, IG, PAIR>(a, st);               \
    case 96: return launch_gemm_inst<DTA, DTW, 96, IG, PAIR>(a, st);               \
    case 128: return launch_gemm_inst<DTA, DTW, 128, IG, PAIR>(a, st);             \
    case 160: return launch_gemm_inst<DTA, DTW, 160, IG, PAIR>(a, st);             \
    default: return hipErrorInvalidValue;                                          \
  }

}  // namespace aih
