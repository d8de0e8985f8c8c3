// conv_pw_narrow.h -- launch interface of the pointwise conv with <= 4 output channels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "aih_device.h"

namespace aih {

// Weight vector vi of the packed narrow weights (one column group: vector
// (kg, j) -- input channels 4kg..4kg+3 of output channel j -- at kg * 4 + j,
// pack.rs:95) in fp32.
template <int DTA, int DTW>
__device__ __forceinline__ f32x4 narrow_w4(const void *w, size_t vi) {
  if constexpr (DTW == DT_F32) return reinterpret_cast<const f32x4 *>(w)[vi];
  else return unpack4<DTW>(reinterpret_cast<const u32x2 *>(w)[vi]);
}

// One input group's contribution to one output channel: the four products
// as one fixed chain of fused multiply-adds. Shared by pw_narrow_kernel and
// the head joined to an inverted-residual block (ir_split_impl.h), so both
// sum the same products the same way.
__device__ __forceinline__ float narrow_dot4(const f32x4 &x, const f32x4 &w) {
  return __builtin_fmaf(x.w, w.w, __builtin_fmaf(x.z, w.z, __builtin_fmaf(x.y, w.y, x.x * w.x)));
}

struct PwNarrowArgs {
  const void *x, *w, *bias, *res;
  void *y;
  uint32_t M;    // pixels over the whole batch
  uint32_t KG;   // input kg (4-channel groups) used
  uint32_t KGX;  // kg per input pixel (the input's pixel stride)
  int32_t act, has_res;
};

// Largest K (in kg) the narrow route takes (one group of G lanes sums a
// pixel's whole K).
constexpr uint32_t kPwNarrowMaxKG = 2048;

// Lanes per pixel for kg input channel groups: 16, 4 or 1.
inline uint32_t pw_narrow_group(uint32_t kg) { return kg >= 16 ? 16u : 1u; }

hipError_t launch_pw_narrow(const PwNarrowArgs &a, int dta, int dtw, hipStream_t st);

}  // namespace aih
