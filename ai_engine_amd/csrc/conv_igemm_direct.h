// conv_igemm_direct.h -- launch interface of the 3x3 implicit-GEMM conv with
// at most 64 output channels whose whole weight tensor fits in LDS (the
// activations go from memory straight into MFMA operand registers), also
// launched with one tap for pointwise convs with mid-size K.
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
  uint32_t taps;           // 9 (3x3) or 1 (1x1: the pointwise route)
  uint32_t ncg;            // column groups of NOB * 32 outputs (work items per block)
  const void *w;           // packed [9][KGP][N4][4]
  const void *bias;        // [N4]
  const void *res;         // like y, or null
  void *y;                 // [M][N4]
  uint32_t KGP, N4;
  uint32_t M, OHW, OW, IH, IW, S, D;
  int32_t PT, PL;
  uint32_t nblk;           // 32-pixel blocks
  int32_t act, has_res;
  uint32_t nxcd;           // XCDs of the device (workgroup remap)
  FastDiv fd_ohw, fd_ow;
  uint32_t st_off;         // LDS byte offset of the output staging rows, 0: none (set by the launch)
};

// Threads of one workgroup (the weights in LDS are shared by its wavefronts).
constexpr uint32_t kIgDirectThreads = 512;
// Most MFMA K steps per tap the kernel takes: 10 units of 16 bytes per lane
// half (80 fp32 / 160 16-bit input channels).
constexpr uint32_t kIgDirectMaxSteps = 10;

// Step counts of the pointwise (1x1) instantiations: a call runs the
// smallest one that holds its steps (the extra steps read zero weights and
// activations).
constexpr uint32_t kPwLdsSteps[5] = {8, 12, 16, 24, 32};
inline uint32_t pw_lds_steps(uint32_t nj) {
  for (uint32_t s : kPwLdsSteps)
    if (nj <= s) return s;
  return 0;
}

// Output columns per wavefront (NOB blocks of 32) and column groups: N4 <=
// 32 -> one block; <= 64 -> two; beyond (1x1 only, <= 256) -> groups of four
// blocks where N4 is a multiple of 128 (each activation load feeds twice the
// MFMAs of a two-block group), else of two; one group per work item.
inline uint32_t ig_direct_nob(uint32_t N4) { return N4 <= 32 ? 1u : N4 > 64 && N4 % 128 == 0 ? 4u : 2u; }
inline uint32_t ig_direct_ncg(uint32_t N4) {
  return N4 <= 64 ? 1u : (N4 + 32 * ig_direct_nob(N4) - 1) / (32 * ig_direct_nob(N4));
}

// LDS bytes of a launch: the weights as [taps][nj][2][ncg * NOB * 32]
// 16-byte units, then the fp32 biases of those columns (nj: the
// instantiation's steps per tap).
inline uint32_t ig_direct_lds_bytes(uint32_t taps, uint32_t nj, uint32_t N4) {
  const uint32_t cols = ig_direct_ncg(N4) * ig_direct_nob(N4) * 32u;
  if (taps == 1) nj = pw_lds_steps(nj);
  return taps * nj * 2u * cols * 16u + cols * 4u;
}

// Workgroups of a launch: one per 8 work items (a block of 32 pixels times
// a column group), at most one per CU of the current device. A second
// resident workgroup per CU (when registers and LDS allow it) measured
// slower on every shape tried: its extra loads in flight contend for the
// same caches (3x3 16 -> 32 stride 2 at 160x288 batch 32, fp32: 62.0 us
// with two per CU, 57.6 us with one).
inline uint32_t ig_direct_grid(uint32_t nblk, uint32_t nj, uint32_t N4) {
  (void)nj;
  const uint64_t items = (uint64_t)nblk * ig_direct_ncg(N4);
  const uint64_t want = (items + kIgDirectThreads / 64 - 1) / (kIgDirectThreads / 64);
  const uint64_t cus = device_cus();
  return (uint32_t)(want < cus ? want : cus);
}

hipError_t launch_ig_direct(const IgDirectArgs &a, int dt, hipStream_t st);

}  // namespace aih
