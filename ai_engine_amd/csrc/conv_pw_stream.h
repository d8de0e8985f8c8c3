// conv_pw_stream.h -- launch interface of the fp32 pointwise conv GEMM with
// operands streamed through LDS by DMA (buffer loads straight into LDS), for
// long K over many pixels (960 -> 160 at 10x18, batch 256).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace aih {

struct PwStreamArgs {
  const void *x;        // [M][KG] 16-byte units (4 fp32 channels)
  const void *w;        // [KGP][N4] 16-byte units (packed 1x1 weights)
  const void *bias;     // [N4] fp32
  const void *res;      // [M][N4] fp32, or null
  void *y;              // [M][N4] fp32
  uint32_t x_bytes;     // bytes of x (< 2 GiB)
  uint32_t w_bytes;     // bytes of w (< 2 GiB)
  uint32_t M;           // pixels over the whole batch
  uint32_t KG;          // input kg (4-channel groups) per pixel
  uint32_t N4;          // output channels padded to 4
  uint32_t mtiles, ntiles;
  int32_t act, has_res;
  uint32_t nxcd;        // XCDs of the device (workgroup remap)
};

// One instantiation: WM x WN wavefronts, each 32 pixels x TN 32-channel
// blocks; a tile is 32 WM pixels x 32 WN TN channels; NST stages of 16
// channels in flight.
struct PwStreamShape {
  uint32_t wm, wn, tn, nst;
};

// The instantiations, in the order the planner tries them: 96-pixel tiles,
// two stages. On 960 -> 160 at 10x18 batch 256 (fp32) 96 x 160 tiles ran
// 126.8 us with two stages, 129.9 / 130.3 us with three / four; 64 x 160
// tiles 148-192 us (three workgroups of 10 wavefronts per CU contend more
// than two of 15), 32 x 160 tiles 154.8 us, one wavefront column of five
// blocks (32 x 160 per wavefront) 158-167 us.
constexpr PwStreamShape kPwStreamShapes[] = {
    {3, 5, 1, 2},  // 96 x 160
    {3, 4, 1, 2},  // 96 x 128
    {3, 3, 1, 2},  // 96 x 96
    {3, 2, 1, 2},  // 96 x 64
};

inline uint32_t pw_stream_bm(const PwStreamShape &s) { return 32 * s.wm; }
inline uint32_t pw_stream_bn(const PwStreamShape &s) { return 32 * s.wn * s.tn; }
// LDS bytes: NST stages of BM pixel rows and BN weight columns, 64 bytes each.
inline uint32_t pw_stream_lds(const PwStreamShape &s) { return s.nst * (pw_stream_bm(s) + pw_stream_bn(s)) * 64; }

// Whether the kernel takes a call: fp32 activations and weights, whole
// buffers below 2 GiB (32-bit buffer offsets). shape: the instantiation.
hipError_t launch_pw_stream(const PwStreamArgs &a, const PwStreamShape &shape, hipStream_t st);

}  // namespace aih
