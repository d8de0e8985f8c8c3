// conv_pw_direct.h -- launch interface of the pointwise conv with short K and
// at most 64 output channels (operands straight from memory into MFMA
// registers, no LDS).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace aih {

struct PwDirectArgs {
  const void *x, *w, *bias, *res;
  void *y;
  uint32_t M;     // pixels over the whole batch
  uint32_t KG;    // input kg (4-channel groups) per pixel (the input's pixel stride)
  uint32_t N4;    // output channels padded to 4 (the weights' and the output's column count)
  uint32_t nblk;  // 32-pixel blocks
  int32_t act, has_res;
};

// Largest K (channels) and N4 the kernel takes: its operands of one 32-pixel
// block stay in registers.
constexpr uint32_t kPwDirectMaxK16 = 128, kPwDirectMaxK32 = 64, kPwDirectMaxN4 = 64;

// Workgroups of a launch over nblk 32-pixel blocks and their wavefronts:
// fewer blocks than four per CU run one wavefront (one block) per
// workgroup, so every CU gets work; otherwise four wavefronts per
// workgroup, at most 8 workgroups per CU, blocks taken grid-stride.
inline uint32_t pw_direct_waves_per_group(uint32_t nblk, uint32_t cus) { return nblk < 4u * cus ? 1u : 4u; }

// grid_out non-null: only the launch's workgroup count is computed (plans).
hipError_t launch_pw_direct(const PwDirectArgs &a, int dt, hipStream_t st, uint32_t *grid_out = nullptr);

}  // namespace aih
