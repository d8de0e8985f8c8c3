// conv_stem.h -- launch interface of the 3x3 conv over images of <= 3 channels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "aih_device.h"

namespace aih {

struct StemArgs {
  const void *x;     // [N][IH][IW][4] NHWC-C4, channels >= cin zero
  const void *w;     // packed [9][KGP][CO/4][4][4]
  const void *bias;  // [CO]
  const void *res;   // like y, or null
  void *y;           // [N][OH][OW][CO]
  uint32_t IH, IW, OHW, OW, S;
  int32_t PT, PL;
  uint32_t CO, KGP;
  uint32_t M, nblocks;  // output pixels over the batch, 32-pixel blocks
  int32_t act, has_res;
  FastDiv fd_ohw, fd_ow;
  uint32_t cin_f32;  // 0: x is NHWC-C4 in the dtype; 1..3: x is logical NHWC fp32 with
                     // that many channels per pixel, rounded to the dtype as it is read
  uint32_t x_bytes;  // bytes of x when cin_f32 != 0 (< 2 GiB)
  uint32_t nxcd;     // XCDs of the device (workgroup remap)
};

// grid_out non-null: only the launch's workgroup count is computed (plans).
hipError_t launch_conv_stem(const StemArgs &a, int dt, hipStream_t st, uint32_t *grid_out = nullptr);

}  // namespace aih
