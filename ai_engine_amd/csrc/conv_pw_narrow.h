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

// Largest K (in kg) the kernel stages in LDS.
constexpr uint32_t kPwNarrowMaxKG = 2048;

hipError_t launch_pw_narrow(const PwNarrowArgs &a, int dta, int dtw, hipStream_t st);

}  // namespace aih
