// conv_pw_narrow.h -- launch interface of the pointwise conv with <= 4 output channels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace aih {

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
inline uint32_t pw_narrow_group(uint32_t kg) { return kg >= 16 ? 16u : kg >= 4 ? 4u : 1u; }

hipError_t launch_pw_narrow(const PwNarrowArgs &a, int dta, int dtw, hipStream_t st);

}  // namespace aih
