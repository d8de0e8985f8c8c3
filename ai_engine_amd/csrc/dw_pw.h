// dw_pw.h -- launch interface of the fused depthwise -> pointwise kernel: a
// depthwise KxK conv (+ act) whose only reader is a 1x1 conv (+ act, +
// residual), in one launch, the depthwise output never stored.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "aih_device.h"

namespace aih {

// 16-byte units of one chunk per halo pixel: 4, i.e. 16 fp32 channels or 32
// 16-bit ones (fp32: 32-channel chunks, whole 128-byte lines, measured
// slower: twice the LDS per buffer halves the resident workgroups, and a
// channel count such as 44 pads its last chunk by a third). In LDS a halo pixel takes one
// more unit, the pad: an odd number of units puts the 16 consecutive pixels
// one ds_read_b128 reads in distinct banks.
constexpr int kDpUnits = 4;
// Most 64-slot rows of the halo region one wavefront copies per chunk (its
// slot offsets stay in registers for the whole launch): 10 at stride 1 (the
// shapes the planner tries need at most 9), 24 at stride 2.
constexpr uint32_t dwpw_slots(uint32_t s) { return s == 1 ? 10u : 24u; }

struct DwPwArgs {
  const void *x;    // depthwise input [N][IH][IW][C] (C a multiple of 4)
  const void *wd;   // depthwise weights [K*K][C]
  const void *bd;   // depthwise bias [C]
  const void *wp;   // pointwise weights, packed [KGP][CO4][4]
  const void *bp;   // pointwise bias [CO4]
  const void *res;  // [N][OH][OW][CO4] or null
  void *y;          // [N][OH][OW][CO4]
  uint32_t img_bytes;  // bytes of one input image
  uint32_t IH, IW, C, OH, OW, CO4, KGP;
  int32_t PT, PL;
  uint32_t TH, TW;   // output tile: wy * nb rows (nb per wavefront), wx * 16 columns
  uint32_t wx;       // wavefronts across the tile
  uint32_t HH, HW;   // halo rows / columns of the tile
  uint32_t HWE;      // stride 2: columns of the even half (ceil(HW / 2)); halo columns are stored even first
  uint32_t tiles_x, per_img, ntiles;
  FastDiv fd_pi, fd_tx, fd_hw;
  uint32_t nchunks;    // chunks of kDpUnits 16-byte units (4 fp32 / 8 16-bit channels each) of C
  uint32_t xrows;      // 64-slot rows (1 KB) of the halo region: HH * HW * (U + 1) slots rounded up
  uint32_t buf_bytes;  // one LDS chunk buffer
  uint32_t off_wd;     // inside a buffer: depthwise weights [K*K][U units], bias [U], pointwise weights [U][COP][4]
  int32_t act_d, act_p, has_res;
  uint32_t nxcd;
};

struct DwPwPlan {
  uint32_t wx, wy, nb, TH, TW, HH, HW, HWE;
  uint32_t tiles_x, tiles_y, ntiles;
  uint32_t xrows, buf_bytes, lds, occ, grid;
};

// Output-channel blocks of 16 (NO) an instantiation exists for.
inline bool dwpw_has_cout(uint32_t cout) { return cout >= 1 && cout <= 64; }
inline uint32_t dwpw_no(uint32_t cout) { return (cout + 15) / 16; }

// 64-slot rows of the halo region of a chunk buffer for a halo of hh x hw pixels.
inline uint32_t dwpw_xrows(uint32_t hh, uint32_t hw) {
  return (hh * hw * (kDpUnits + 1) + 63) / 64;
}

// LDS bytes of one chunk buffer: the halo region, then the weights.
inline uint32_t dwpw_buf_bytes(uint32_t k, uint32_t s, uint32_t hh, uint32_t hw, uint32_t cout) {
  const uint32_t u = kDpUnits, cop = dwpw_no(cout) * 16;
  return dwpw_xrows(hh, hw) * 1024 + (k * k * u + u + u * cop) * 16;
}

// rows: output rows per wavefront (2 or 4).
hipError_t launch_dw_pw(const DwPwArgs &a, int dt, uint32_t k, uint32_t s, uint32_t rows, uint32_t waves,
                        uint32_t lds, uint32_t grid, hipStream_t st);
// The 16-bit instantiations (dw_pw_f16.hip, dw_pw_bf16.hip). occ: -2 no
// instantiation, -1 no device to ask, else workgroups per CU.
hipError_t launch_dw_pw_f16(const DwPwArgs &a, uint32_t k, uint32_t s, uint32_t rows, uint32_t waves, uint32_t lds,
                            uint32_t grid, hipStream_t st);
hipError_t launch_dw_pw_bf16(const DwPwArgs &a, uint32_t k, uint32_t s, uint32_t rows, uint32_t waves, uint32_t lds,
                             uint32_t grid, hipStream_t st);
int dw_pw_occ_f16(uint32_t k, uint32_t s, uint32_t no, uint32_t rows, bool cl, uint32_t waves, uint32_t lds);
int dw_pw_occ_bf16(uint32_t k, uint32_t s, uint32_t no, uint32_t rows, bool cl, uint32_t waves, uint32_t lds);
// cl: both activations clamp-type (the instantiation launch_dw_pw runs for them).
int dw_pw_occupancy(int dt, uint32_t k, uint32_t s, uint32_t cout, uint32_t rows, bool cl, uint32_t waves,
                    uint32_t lds);

}  // namespace aih
