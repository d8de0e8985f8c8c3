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

// ---- the 16-bit stem's MFMA operands, shared with the block kernel that
// computes the stem inside its halo loads (ir_wave_impl.h) ----
//
// 4 K per tap (the fourth channel zero), 3 steps of v_mfma_f32_32x32x16;
// the two lane halves hold different taps: load slot i of lane half h holds
// tap stem_slot_tap(h, i) (ky*3 + kx; 9 = none). Both halves of a slot read
// the same input row at neighbouring columns but one (slot 3), so one load
// instruction touches about as many cache lines as a single tap would; slots
// 2s and 2s + 1 of a half feed MFMA step s.
__host__ __device__ constexpr int stem_slot_tap(int h, int i) {
  constexpr int t[2][6] = {{0, 3, 6, 2, 8, 9}, {1, 4, 7, 5, 9, 9}};
  return t[h][i];
}

// The accumulator of a 32x32 block starting at the bias: lane (pixel, half
// lh) holds channels 8q + 4lh .. + 3 in elements 4q .. 4q + 3, b[q] those
// channels' bias.
__device__ __forceinline__ f32x16 stem_acc_init(const f32x4 (&b)[4]) {
  return f32x16{b[0].x, b[0].y, b[0].z, b[0].w, b[1].x, b[1].y, b[1].z, b[1].w,
                b[2].x, b[2].y, b[2].z, b[2].w, b[3].x, b[3].y, b[3].z, b[3].w};
}

// A operand of output channel o (lane row), lane half lh, step s: K =
// s*16 + lh*8 + j, j < 4 the channels (ic 3 zero) of tap stem_slot_tap(lh,
// 2s), j >= 4 those of stem_slot_tap(lh, 2s + 1), from the packed weights:
// element (tap, kg 0, n = o, comp = ic) at ((tap*KGP)*NG + o/4)*16 + (o%4)*4
// + ic (pack.rs:95), 16-bit storage bits.
__device__ __forceinline__ u32x4 stem_a16(const void *w, uint32_t KGP, uint32_t NG, uint32_t o, int lh, int s) {
  auto wt = [&](int tap, int ic) -> uint32_t {
    if (tap >= 9 || ic >= 3) return 0u;
    return reinterpret_cast<const uint16_t *>(w)[((size_t)tap * KGP * NG + o / 4) * 16 + (o % 4) * 4 + ic];
  };
  const int t = lh ? stem_slot_tap(1, 2 * s) : stem_slot_tap(0, 2 * s);
  const int u = lh ? stem_slot_tap(1, 2 * s + 1) : stem_slot_tap(0, 2 * s + 1);
  return u32x4{wt(t, 0) | (wt(t, 1) << 16), wt(t, 2), wt(u, 0) | (wt(u, 1) << 16), wt(u, 2)};
}

}  // namespace aih
