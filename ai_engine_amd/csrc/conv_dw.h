// conv_dw.h -- launch interface of the depthwise conv and device pack kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace aih {

struct DwArgs {
  const void *x, *w, *bias, *res;
  void *y;
  uint32_t N, IH, IW, OH, OW, CG;
  uint32_t K, S, D;
  int32_t PT, PL;
  int32_t act, has_res;
  uint32_t nxcd;  // XCDs of the device (workgroup remap)
};

hipError_t launch_conv_dw(const DwArgs &a, int dt, hipStream_t st);
hipError_t launch_pack_nhwc(const float *x, uint64_t px, uint32_t c, int dt, void *y, hipStream_t st);

}  // namespace aih
