// conv_pw_splitk.h -- launch interface of the one-dispatch split-K pointwise
// conv: small M, long K (the reference's gemm_pw_splitk role, an in-workgroup
// K split with the reduction on chip).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace aih {

struct PwSplitkArgs {
  const void *x, *w, *bias, *res;
  void *y;
  uint32_t M;       // pixels over the whole batch
  uint32_t KG;      // input kg (4-channel groups) per pixel (the input's pixel stride)
  uint32_t N4;      // output channels padded to 4; a multiple of 16
  uint32_t mblk;    // 16-pixel blocks
  uint32_t nblk;    // 16-channel blocks
  uint32_t steps;   // K steps of the whole K (fp32: 4 kg, 16-bit: 8 kg per step)
  uint32_t spw;     // K steps per wavefront (the last one may take fewer)
  int32_t act, has_res;
  uint32_t nxcd;    // XCDs of the device (workgroup remap)
};

// Shapes the kernel is planned for: at most this many pixels (every
// workgroup re-reads its 16 pixels' K and its 16 channels' weights from the
// caches; beyond this the tiled GEMM's reuse wins).
constexpr uint32_t kPwSplitkMaxM = 2048;
// Waves (K chunks) per workgroup that have an instantiation.
constexpr uint32_t kPwSplitkWaves[] = {1, 2, 4, 8, 16};

// K steps of a pointwise conv in this kernel's units.
inline uint32_t pw_splitk_steps(uint32_t kg, bool f32) { return f32 ? (kg + 3) / 4 : (kg + 7) / 8; }

// The policy's chunk count: the most waves (<= 16) that still give every
// wave two K steps.
inline uint32_t pw_splitk_waves(uint32_t steps) {
  uint32_t w = 1;
  while (w < 16 && steps / (2 * w) >= 2) w *= 2;
  return w;
}

hipError_t launch_pw_splitk(const PwSplitkArgs &a, int dt, uint32_t waves, hipStream_t st);

}  // namespace aih
