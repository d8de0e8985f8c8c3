// conv_igemm_direct.h -- launch interface of the 3x3 implicit-GEMM conv with
// at most 64 output channels whose whole weight tensor fits in LDS (the
// activations go from memory straight into MFMA operand registers).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "aih_device.h"

namespace aih {

struct IgDirectArgs {
  const void *src[2];      // input parts (one for a plain input)
  uint32_t src_bytes[2];   // bytes of each part's buffer (< 2 GiB)
  uint32_t stride_u[2];    // pixel stride of each part, in 16-byte units
  uint32_t off_u[2];       // first unit of each part inside its pixel
  uint32_t nu[2];          // 16-byte units of each part per pixel
  uint32_t kg_first[2];    // first kg (of the packed weights) of each part
  uint32_t nj0, nj;        // MFMA K steps per tap: of part 0, of all parts
  const void *w;           // packed [9][KGP][N4][4]
  const void *bias;        // [N4]
  const void *res;         // like y, or null
  void *y;                 // [M][N4]
  uint32_t KGP, N4;
  uint32_t M, OHW, OW, IH, IW, S, D;
  int32_t PT, PL;
  uint32_t nblk;           // 32-pixel blocks
  int32_t act, has_res;
  FastDiv fd_ohw, fd_ow;
};

// Threads of one workgroup (the weights in LDS are shared by its wavefronts).
constexpr uint32_t kIgDirectThreads = 512;
// Most MFMA K steps per tap the kernel takes: 8 units of 16 bytes per lane
// half (64 fp32 / 128 16-bit input channels).
constexpr uint32_t kIgDirectMaxSteps = 8;

// LDS bytes of a launch: the weights as [9][nj][2][NOB*32] 16-byte units,
// then NOB*32 fp32 biases.
inline uint32_t ig_direct_lds_bytes(uint32_t nj, uint32_t N4) {
  const uint32_t nob = N4 <= 32 ? 1u : 2u;
  return 9u * nj * 2u * nob * 32u * 16u + nob * 32u * 4u;
}

// Workgroups of a launch: one per 8 blocks, at most what stays resident --
// two workgroups per CU when their LDS allows and the kernel keeps to 128
// VGPRs (one 32-column block: <= 124), one otherwise (two blocks: 115-154).
inline uint32_t ig_direct_grid(uint32_t nblk, uint32_t nj, uint32_t N4) {
  const uint32_t lds = ig_direct_lds_bytes(nj, N4);
  const uint32_t occ = N4 <= 32 && lds * 2 <= 160u * 1024u ? 2u : 1u;
  const uint64_t want = ((uint64_t)nblk + kIgDirectThreads / 64 - 1) / (kIgDirectThreads / 64);
  return (uint32_t)(want < 256ull * occ ? want : 256ull * occ);
}

hipError_t launch_ig_direct(const IgDirectArgs &a, int dt, hipStream_t st);

}  // namespace aih
