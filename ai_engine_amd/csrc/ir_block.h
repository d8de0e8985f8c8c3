// ir_block.h -- launch interface of the fused inverted-residual block kernel.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "aih_device.h"

namespace aih {

// One inverted-residual block: 1x1 expand (C -> E) + act, depthwise 3x3
// (stride S) + act, 1x1 project (E -> CO) + act (+ residual), all tensors
// NHWC-C4 with the batch outermost, weights in the converter's packed layouts.
struct IrArgs {
  const void *x;         // [N][IH][IW][C]
  const void *we, *be;   // expand weights [C/4][E][4], bias [E]
  const void *wd, *bd;   // depthwise weights [9][E/4][4], bias [E]
  const void *wp, *bp;   // project weights [E/4][CO][4], bias [CO]
  const void *res;       // [N][OH][OW][CO] or null
  void *y;               // [N][OH][OW][CO]
  uint32_t N, IH, IW, OH, OW;
  uint32_t C, E, CO;
  uint32_t COP;          // CO rounded up to 32: the projection's MFMA width and LDS weight pitch
  uint32_t S;
  int32_t PT, PL;
  uint32_t TH, TW;       // output tile
  uint32_t HH, HW;       // input (halo) tile: (TH-1)*S+3 x (TW-1)*S+3
  uint32_t NPI, NPB;     // 32-pixel blocks of the halo tile / of the output tile
  uint32_t EC;           // expanded channels per chunk (multiple of 32)
  uint32_t resident;     // 1: all E channels' weights stay in LDS for every tile
  uint32_t tiles_y, tiles_x, ntiles;
  int32_t act_e, act_d, act_p, has_res;
  int32_t mask_e;        // act_e(0) != 0: expanded halo pixels outside the image are masked to 0
  int32_t clamp_acts;    // all three activations clamp-type (act_is_clamp): branch-free instantiation
  uint32_t nxcd;         // XCDs of the device (workgroup remap)
  uint32_t lds_x, lds_xe, lds_we, lds_wp, lds_sm, lds_bp;  // LDS byte offsets
  // divisors the kernel uses, prepared on the host
  FastDiv fd_rpx;              // 16-byte items per LDS input row (vectors per pixel + 1)
  FastDiv fd_hw, fd_tw;        // halo tile width, output tile width
  FastDiv fd_tx, fd_pi;        // tiles per row, tiles per image
};

// Tile / chunk geometry of one launch, chosen by ir_plan.
struct IrPlan {
  uint32_t TH, TW, HH, HW, NPI, NPB, EC, resident;
  uint32_t tiles_y, tiles_x, ntiles;
  uint32_t lds_x, lds_xe, lds_we, lds_wp, lds_sm, lds_bp, lds;  // LDS byte offsets and total
  uint32_t occ, grid;  // workgroups per CU, launched workgroups
};

// Chooses the tile and chunk geometry for an inverted-residual block
// (depthwise 3x3, stride S). Returns nullptr on success, otherwise the reason
// the block cannot run fused.
// tile_h / tile_w / ec force that part of the geometry when non-zero;
// weights (enum aih_ir_weights) forces resident or streamed weights.
// cl: every activation is clamp-type (selects the instantiation whose register
// use bounds the occupancy).
const char *ir_plan(uint32_t N, uint32_t IH, uint32_t IW, uint32_t OH, uint32_t OW, uint32_t C, uint32_t E,
                    uint32_t CO, uint32_t S, int dt, bool cl, uint32_t tile_h, uint32_t tile_w, uint32_t ec,
                    int32_t weights, IrPlan *p);

hipError_t launch_ir_block(const IrArgs &a, int dt, uint32_t lds, uint32_t grid, hipStream_t st);

// ---- the one-tile-per-wavefront kernel (ir_wave_impl.h) ----

constexpr int IRW_THREADS = 512;              // the most threads a split-kernel workgroup has (8 wavefronts)
// The most wavefronts a wave-kernel workgroup of a shape (KE = C / 16, NPI
// halo blocks, NOB = COP / 32) has: 12 -- three per SIMD, one workgroup a
// CU sharing one resident copy of the weights -- where the shape's registers
// fit 168 VGPRs (the stride-1 tiles of 32-, 48- and 64-channel blocks), else
// 8.
__host__ __device__ constexpr uint32_t irw_max_waves(uint32_t ke, uint32_t npi, uint32_t nob) {
  return npi == 2 && ((nob == 2 && (ke == 3 || ke == 4)) || (nob == 1 && ke == 2)) ? 12u : 8u;
}
// A wavefront's expanded chunk in LDS: four planes of 8 channels (16 bytes a
// halo pixel), plane h holding channels 8h .. 8h + 7 of every halo pixel in
// turn -- 64 bytes a pixel. (The depthwise reads 16-pixel groups of one
// plane; measured on gfx950, these reads cost 6.5 LDS cycles per wavefront
// instruction against 8.8 - 9.6 for rows of 64 + 16 bytes a pixel.)
constexpr uint32_t IRW_XPIX = 32 * 2;         // bytes of one halo pixel over the four planes
// Per chunk, after the expand and project weights: the 9 depthwise taps
// (32 16-bit channels each), a run of 32 zeros (the partner of the ninth tap
// in the depthwise MFMAs), the depthwise bias and the expand bias.
constexpr uint32_t IRW_TAPS_ZERO = 9 * 32 * 2;
constexpr uint32_t IRW_BD = 10 * 32 * 2;
constexpr uint32_t IRW_BE = 11 * 32 * 2;
constexpr uint32_t IRW_SMB = 12 * 32 * 2;

struct IrWaveArgs {
  const void *x;         // [N][IH][IW][C]
  const void *we, *be;   // expand weights [C/4][E][4], bias [E]
  const void *wd, *bd;   // depthwise weights [9][E/4][4], bias [E]
  const void *wp, *bp;   // project weights [E/4][CO][4], bias [CO]
  const void *res;       // [N][OH][OW][CO] or null
  void *y;               // [N][OH][OW][CO]
  uint32_t N, IH, IW, OH, OW;
  uint32_t C, E, CO, S;
  uint32_t COP;             // CO rounded up to 32: the projection's MFMA width and LDS weight pitch
  int32_t PT, PL;
  uint32_t TH, TW, HH, HW;  // output tile (<= 32 pixels), input (halo) tile
  uint32_t tiles_y, tiles_x, ntiles;
  uint32_t resident;        // 1: every chunk's weights stay in LDS; 0: two streamed slots
  int32_t act_e, act_d, act_p, has_res;
  uint32_t nxcd;            // XCDs of the device (workgroup remap)
  uint32_t lds_w, lds_bp, lds_xe;  // LDS byte offsets: weight slots, fp32 projection bias, expanded regions
  uint32_t lds_red;                // split kernel: projection partial sums (over the regions below)
  uint32_t lds_x;                  // split kernel: the tile's input halo
  FastDiv fd_hw, fd_tw, fd_tx, fd_pi;
  // ir_wave_stem_kernel only: the block's input (and residual) is the output
  // of a 3x3 stem conv over a 3-channel fp32 image, computed per halo pixel
  // instead of read (x and res unused)
  const void *sx;                  // the image [N][SIH][SIW][3], fp32, < 2 GiB
  const void *sw, *sb;             // stem weights (packed, the storage dtype) and bias [C]
  uint32_t SIH, SIW, SS, sx_bytes; // image size, stem stride, bytes of sx
  int32_t SPT, SPL, act_s;         // stem padding (top, left), activation (clamp-type)
  uint32_t lds_stem, lds_res;      // LDS: stem A operands + fp32 bias; per-wavefront residual stashes
  uint32_t lds_next;               // wave kernel, resident weights: the workgroup's next-tile counter (16 bytes)
  // split kernel only: a pointwise conv with <= 4 output channels (one
  // NHWC-C4 vector a pixel) reading the block's output -- the segmentation
  // head -- joined to it; y may then be null (the block's output not stored)
  const void *hw, *hb;             // head weights (packed, kg * 4 + j), bias [4]
  void *hy;                        // head output [N][OH][OW][4], or null: no head
  int32_t act_h;                   // head activation
  uint32_t lds_head;               // LDS: the head's per-lane partial sums (IRW_HEAD_LDS bytes)
};

// LDS of the head joined to a split-kernel block: per 16-pixel group and
// pixel, the 16 lanes' partial sums of pw_narrow_kernel (four fp32 each).
constexpr uint32_t IRW_HEAD_LDS = 2 * 16 * 16 * 16;

// LDS of the stem-fused launch beyond the block's own: the stem's A operands
// (3 MFMA steps x 64 lanes x 16 bytes) and fp32 bias (32 channels), and per
// wavefront the tile's stem outputs (<= 32 pixels x 32 16-bit channels),
// the block's residual.
constexpr uint32_t IRW_STEM_LDS = 3 * 64 * 16 + 32 * 4;
constexpr uint32_t IRW_RES_STASH = 32 * 32 * 2;

// Bytes of one chunk's weight slot: expand [C/4][32][4], project [8][COP][4]
// (channels CO..COP zero), then IRW_SMB bytes of depthwise taps and biases
// (16-bit elements).
__host__ __device__ inline uint32_t irw_slot_bytes(uint32_t C, uint32_t COP) { return 64 * C + 64 * COP + IRW_SMB; }

// The projection width the kernels compute: cout (a multiple of 16) rounded
// up to whole 32-channel MFMA blocks.
__host__ __device__ inline uint32_t ir_cop(uint32_t CO) { return (CO + 31) / 32 * 32; }

// Tile, weight placement and LDS layout of one launch of the wave kernel
// (split = 0: a tile per wavefront) or of the split kernel (split = 1: a
// tile per workgroup, its chunks divided among the wavefronts).
struct IrWavePlan {
  uint32_t split;
  uint32_t deep;                        // split kernel: operands prefetched a whole chunk ahead
  uint32_t TH, TW, HH, HW, NPI, resident;
  uint32_t waves;                       // wavefronts per workgroup (wave: 2, 4, 8 or 12; split: 1, 2, 4 or 8)
  uint32_t tiles_y, tiles_x, ntiles;
  uint32_t lds_w, lds_bp, lds_xe, lds_red, lds_x, lds;  // LDS byte offsets and total
  uint32_t lds_stem, lds_res;           // stem-fused launch: stem tables, residual stashes
  uint32_t lds_next;                    // wave kernel, resident weights: next-tile counter
  uint32_t lds_head;                    // split kernel with a joined head: its partial sums
  uint32_t occ, grid;                   // workgroups per CU, launched workgroups
};

// Split kernel LDS: the tile's halo (NPI x 32 rows of C channels + 16
// bytes), per wavefront its expanded chunk and its two-slot ring of
// depthwise taps and biases; partial sums: NOB blocks of 32 x 32 fp32 for
// each of up to four wavefronts (eight add theirs in pairs first), over the
// rest once it is done with.
constexpr uint32_t IRS_RING = 2 * IRW_SMB;
constexpr uint32_t IRS_RED_BLOCK = 32 * 32 * 4;

// Chooses between the wave kernel and the split kernel (kernel: enum
// aih_ir_kernel, AUTO for the cheaper estimate), the tile (<= 32 output
// pixels, halo within NPI blocks of an instantiation), the wave kernel's
// weight placement (resident when all chunks fit in LDS next to the
// wavefronts' expanded regions) and the wavefronts per workgroup (waves: 0 =
// the plan's choice). Returns nullptr, or the reason the block cannot run on
// these kernels (dtype, activations, widths without an instantiation, LDS).
// rl: the expand and depthwise activations are both ReLU (selects the
// instantiation whose register use bounds the occupancy). stem: the plan of
// the stem-fused launch (ir_wave_stem_kernel: the wave kernel's 32 -> E -> 32
// stride-1 shape with ReLU inside, its LDS grown by the stem tables and the
// wavefronts' residual stashes). head: the split kernel's plan with the
// joined head's LDS (split plans only).
const char *irw_plan(uint32_t N, uint32_t IH, uint32_t IW, uint32_t OH, uint32_t OW, uint32_t C, uint32_t E,
                     uint32_t CO, uint32_t S, int dt, bool cl, bool rl, uint32_t tile_h, uint32_t tile_w,
                     int32_t weights, int32_t kernel, uint32_t waves, IrWavePlan *p, bool stem = false,
                     bool head = false);

hipError_t launch_ir_wave(const IrWaveArgs &a, int dt, const IrWavePlan &p, hipStream_t st);
hipError_t launch_ir_wave_stem(const IrWaveArgs &a, int dt, const IrWavePlan &p, hipStream_t st);

}  // namespace aih
