// conv_dw.hip -- depthwise KxK conv and the device-side NHWC -> NHWC-C4 pack.
//
// Depthwise is HBM-bound (2 flops per weight per pixel, no reuse across
// channels): the kernel streams NHWC-C4 with one 4-channel vector per thread,
// consecutive threads on consecutive channel groups of a pixel, so every
// wavefront touches contiguous memory. Each thread computes PX horizontally
// adjacent output pixels of one channel group so that the tap weights (read
// once per thread) are reused PX times. The arithmetic follows the reference
// depthwise path (crates/ai-cpu/src/kernels/dw.rs:40-204, ConvDwSpec
// crates/ai-gpu/src/kernels/conv_dw.rs:21-216): acc = bias, then taps in
// (ky, kx) order, then act, then + residual.
#include "aih_device.h"
#include "conv_dw.h"

namespace aih {

template <int DT, int PX>
__global__ __launch_bounds__(256) void conv_dw_kernel(DwArgs a) {
  const uint32_t cg = a.CG;
  const uint64_t gid = (uint64_t)blockIdx.x * 256 + threadIdx.x;
  const uint32_t owb = (a.OW + PX - 1) / PX;  // pixel blocks per output row
  const uint64_t total = (uint64_t)a.N * a.OH * owb * cg;
  if (gid >= total) return;
  const uint32_t g = (uint32_t)(gid % cg);
  uint64_t r = gid / cg;
  const uint32_t xb = (uint32_t)(r % owb);
  r /= owb;
  const uint32_t oy = (uint32_t)(r % a.OH);
  const uint32_t img = (uint32_t)(r / a.OH);
  const uint32_t ox0 = xb * PX;

  const f32x4 b = Vec4IO<DT>::load(a.bias, g);
  f32x4 acc[PX];
#pragma unroll
  for (int p = 0; p < PX; ++p) acc[p] = b;

  const size_t img_base = (size_t)img * a.IH * a.IW;
  for (uint32_t ky = 0; ky < a.K; ++ky) {
    const int32_t iy = (int32_t)(oy * a.S + ky * a.D) - a.PT;
    if ((uint32_t)iy >= a.IH) continue;
    const size_t row = img_base + (size_t)iy * a.IW;
    for (uint32_t kx = 0; kx < a.K; ++kx) {
      const f32x4 w = Vec4IO<DT>::load(a.w, (size_t)(ky * a.K + kx) * cg + g);
#pragma unroll
      for (int p = 0; p < PX; ++p) {
        const int32_t ix = (int32_t)((ox0 + p) * a.S + kx * a.D) - a.PL;
        if ((uint32_t)ix < a.IW && ox0 + p < a.OW) {
          const f32x4 x = Vec4IO<DT>::load(a.x, (row + (uint32_t)ix) * cg + g);
          acc[p] += x * w;
        }
      }
    }
  }
  const size_t orow = ((size_t)img * a.OH + oy) * a.OW;
#pragma unroll
  for (int p = 0; p < PX; ++p) {
    if (ox0 + p >= a.OW) break;
    const size_t vi = (orow + ox0 + p) * cg + g;
    f32x4 v = act_apply4(a.act, acc[p]);
    if (a.has_res) v += Vec4IO<DT>::load(a.res, vi);
    Vec4IO<DT>::store(a.y, vi, v);
  }
}

hipError_t launch_conv_dw(const DwArgs &a, int dt, hipStream_t st) {
  constexpr int PX = 2;
  const uint64_t total = (uint64_t)a.N * a.OH * ((a.OW + PX - 1) / PX) * a.CG;
  const dim3 grid((unsigned)((total + 255) / 256));
  switch (dt) {
    case DT_F32: hipLaunchKernelGGL((conv_dw_kernel<DT_F32, PX>), grid, dim3(256), 0, st, a); break;
    case DT_F16: hipLaunchKernelGGL((conv_dw_kernel<DT_F16, PX>), grid, dim3(256), 0, st, a); break;
    case DT_BF16: hipLaunchKernelGGL((conv_dw_kernel<DT_BF16, PX>), grid, dim3(256), 0, st, a); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

// Logical NHWC fp32 -> NHWC-C4 in DT (zero-filled channel padding); one
// output vec4 per thread.
template <int DT>
__global__ __launch_bounds__(256) void pack_nhwc_kernel(const float *__restrict__ x, uint64_t px, uint32_t c,
                                                        void *y) {
  const uint32_t cg = (c + 3) / 4;
  const uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= px * cg) return;
  const uint64_t p = i / cg;
  const uint32_t g = (uint32_t)(i - p * cg);
  f32x4 v = {};
#pragma unroll
  for (int l = 0; l < 4; ++l) {
    const uint32_t ch = g * 4 + l;
    if (ch < c) v[l] = x[p * c + ch];
  }
  Vec4IO<DT>::store(y, i, v);
}

hipError_t launch_pack_nhwc(const float *x, uint64_t px, uint32_t c, int dt, void *y, hipStream_t st) {
  const uint64_t n = px * ((c + 3) / 4);
  const dim3 grid((unsigned)((n + 255) / 256));
  switch (dt) {
    case DT_F32: hipLaunchKernelGGL(pack_nhwc_kernel<DT_F32>, grid, dim3(256), 0, st, x, px, c, y); break;
    case DT_F16: hipLaunchKernelGGL(pack_nhwc_kernel<DT_F16>, grid, dim3(256), 0, st, x, px, c, y); break;
    case DT_BF16: hipLaunchKernelGGL(pack_nhwc_kernel<DT_BF16>, grid, dim3(256), 0, st, x, px, c, y); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace aih
