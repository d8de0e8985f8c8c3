// conv_dw.hip -- depthwise KxK conv and the device-side NHWC -> NHWC-C4 pack.
//
// Depthwise is HBM-bound (2 flops per weight per pixel, no reuse across
// channels). The arithmetic follows the reference depthwise path
// (crates/ai-cpu/src/kernels/dw.rs:40-204, ConvDwSpec
// crates/ai-gpu/src/kernels/conv_dw.rs:21-216): acc = bias, then the taps in
// (ky, kx) order, then act, then + residual.
//
// conv_dw_strip_kernel (k = 3 or 5, stride 1 or 2, dilation 1): a thread owns
// one 16-byte channel vector (4 fp32 or 8 16-bit channels) of a strip of PX
// horizontally adjacent output pixels. Per kernel row it loads the
// (PX-1)*S + K input columns the strip needs once, with 16-byte loads, and
// reuses each of them for every tap that touches it; consecutive threads take
// consecutive channel vectors of a pixel, so a wavefront reads whole pixel
// rows. conv_dw_kernel is the general fallback (any k, s, dilation).
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
    f32x4 v = act4(act_params(a.act), acc[p]);
    if (a.has_res) v += Vec4IO<DT>::load(a.res, vi);
    Vec4IO<DT>::store(a.y, vi, v);
  }
}

// CV consecutive channels (one 16-byte vector, or 8 bytes for CV = 4 16-bit)
// <-> fp32 registers; idx counts CV-channel vectors.
template <int DT, int CV>
__device__ __forceinline__ void ld_cv(const void *base, size_t idx, float (&out)[CV]) {
  if constexpr (DT == DT_F32) {
    static_assert(CV == 4, "fp32 vectors are 4 channels");
    const f32x4 v = reinterpret_cast<const f32x4 *>(base)[idx];
    out[0] = v.x; out[1] = v.y; out[2] = v.z; out[3] = v.w;
  } else if constexpr (CV == 8) {
    const u32x4 r = reinterpret_cast<const u32x4 *>(base)[idx];
    const f32x4 lo = unpack4<DT>(u32x2{r.x, r.y}), hi = unpack4<DT>(u32x2{r.z, r.w});
    out[0] = lo.x; out[1] = lo.y; out[2] = lo.z; out[3] = lo.w;
    out[4] = hi.x; out[5] = hi.y; out[6] = hi.z; out[7] = hi.w;
  } else {
    const f32x4 v = unpack4<DT>(reinterpret_cast<const u32x2 *>(base)[idx]);
    out[0] = v.x; out[1] = v.y; out[2] = v.z; out[3] = v.w;
  }
}

template <int DT, int CV>
__device__ __forceinline__ void st_cv(void *base, size_t idx, const float (&v)[CV]) {
  if constexpr (DT == DT_F32) {
    reinterpret_cast<f32x4 *>(base)[idx] = f32x4{v[0], v[1], v[2], v[3]};
  } else if constexpr (CV == 8) {
    const u32x2 lo = pack4<DT>(f32x4{v[0], v[1], v[2], v[3]});
    const u32x2 hi = pack4<DT>(f32x4{v[4], v[5], v[6], v[7]});
    reinterpret_cast<u32x4 *>(base)[idx] = u32x4{lo.x, lo.y, hi.x, hi.y};
  } else {
    reinterpret_cast<u32x2 *>(base)[idx] = pack4<DT>(f32x4{v[0], v[1], v[2], v[3]});
  }
}

template <int DT, int CV, int K, int S, int PX>
__global__ __launch_bounds__(256) void conv_dw_strip_kernel(DwArgs a) {
  constexpr int NCOL = (PX - 1) * S + K;  // input columns under one strip
  const uint32_t cgv = a.CG * 4 / CV;     // channel vectors per pixel
  // Workgroups are dealt round-robin to the 8 XCDs; remapping gives each XCD
  // a contiguous run of output rows, so the input rows shared by vertically
  // adjacent outputs are fetched into one L2 instead of one per XCD.
  const uint64_t gid = (uint64_t)xcd_remap(blockIdx.x, gridDim.x, a.nxcd) * 256 + threadIdx.x;
  const uint32_t owb = (a.OW + PX - 1) / PX;
  const uint64_t total = (uint64_t)a.N * a.OH * owb * cgv;
  if (gid >= total) return;
  const uint32_t g = (uint32_t)(gid % cgv);
  uint64_t r = gid / cgv;
  const uint32_t xb = (uint32_t)(r % owb);
  r /= owb;
  const uint32_t oy = (uint32_t)(r % a.OH);
  const uint32_t img = (uint32_t)(r / a.OH);
  const uint32_t ox0 = xb * PX;

  float b[CV];
  ld_cv<DT, CV>(a.bias, g, b);
  float acc[PX][CV];
#pragma unroll
  for (int p = 0; p < PX; ++p)
#pragma unroll
    for (int j = 0; j < CV; ++j) acc[p][j] = b[j];

  const int32_t ix0 = (int32_t)(ox0 * S) - a.PL;
  const Act actp = act_params(a.act);
  const size_t img_base = (size_t)img * a.IH * a.IW;
#pragma unroll
  for (int ky = 0; ky < K; ++ky) {
    const int32_t iy = (int32_t)(oy * S + ky) - a.PT;
    if ((uint32_t)iy >= a.IH) continue;
    const size_t row = img_base + (size_t)iy * a.IW;
    float xv[NCOL][CV];
#pragma unroll
    for (int c = 0; c < NCOL; ++c) {
      const int32_t ix = ix0 + c;
      if ((uint32_t)ix < a.IW) {
        ld_cv<DT, CV>(a.x, (row + (uint32_t)ix) * cgv + g, xv[c]);
      } else {
#pragma unroll
        for (int j = 0; j < CV; ++j) xv[c][j] = 0.0f;
      }
    }
#pragma unroll
    for (int kx = 0; kx < K; ++kx) {
      float w[CV];
      ld_cv<DT, CV>(a.w, (size_t)(ky * K + kx) * cgv + g, w);
#pragma unroll
      for (int p = 0; p < PX; ++p)
#pragma unroll
        for (int j = 0; j < CV; ++j) acc[p][j] += xv[p * S + kx][j] * w[j];
    }
  }
  const size_t orow = ((size_t)img * a.OH + oy) * a.OW;
#pragma unroll
  for (int p = 0; p < PX; ++p) {
    if (ox0 + p >= a.OW) break;
    const size_t vi = (orow + ox0 + p) * cgv + g;
    float v[CV];
#pragma unroll
    for (int j = 0; j < CV; ++j) v[j] = acc[p][j];
    act_array<CV>(actp, v);
    if (a.has_res) {
      float rr[CV];
      ld_cv<DT, CV>(a.res, vi, rr);
#pragma unroll
      for (int j = 0; j < CV; ++j) v[j] += rr[j];
    }
    st_cv<DT, CV>(a.y, vi, v);
  }
}

template <int DT, int CV, int K, int S, int PX>
static hipError_t launch_strip_px(const DwArgs &a, hipStream_t st) {
  const uint64_t total = (uint64_t)a.N * a.OH * ((a.OW + PX - 1) / PX) * (a.CG * 4 / CV);
  const dim3 grid((unsigned)((total + 255) / 256));
  hipLaunchKernelGGL((conv_dw_strip_kernel<DT, CV, K, S, PX>), grid, dim3(256), 0, st, a);
  return hipGetLastError();
}

// Strips of 4 output pixels where that still gives every SIMD four
// wavefronts (64 lanes x 4 x 4 SIMDs per CU); small late layers (10x18 or
// 20x36 outputs) take strips of 2 or 1 pixels instead, so their launches fill
// the GPU rather than leaving most CUs idle with long per-thread tap loops.
template <int DT, int CV, int K, int S>
static hipError_t launch_strip(const DwArgs &a, hipStream_t st) {
  const uint64_t want = (uint64_t)device_cus() * 4 * 4 * 64;
  const uint64_t per_px = (uint64_t)a.N * a.OH * (a.CG * 4 / CV);
  if (per_px * ((a.OW + 3) / 4) >= want) return launch_strip_px<DT, CV, K, S, 4>(a, st);
  if (per_px * ((a.OW + 1) / 2) >= want) return launch_strip_px<DT, CV, K, S, 2>(a, st);
  return launch_strip_px<DT, CV, K, S, 1>(a, st);
}

template <int DT, int CV>
static hipError_t launch_strip_ks(const DwArgs &a, hipStream_t st) {
  if (a.K == 3) return a.S == 1 ? launch_strip<DT, CV, 3, 1>(a, st) : launch_strip<DT, CV, 3, 2>(a, st);
  return a.S == 1 ? launch_strip<DT, CV, 5, 1>(a, st) : launch_strip<DT, CV, 5, 2>(a, st);
}

hipError_t launch_conv_dw(const DwArgs &a, int dt, hipStream_t st) {
  if (a.D == 1 && (a.K == 3 || a.K == 5) && (a.S == 1 || a.S == 2)) {
    // two 4-channel groups per 16-byte vector, unless one-pixel strips of
    // 8-channel vectors still leave the GPU short of threads (small late
    // layers): then 4-channel vectors, twice the threads
    const uint64_t one_px8 = (uint64_t)a.N * a.OH * a.OW * (a.CG / 2);
    const bool cv8 = a.CG % 2 == 0 && one_px8 >= (uint64_t)device_cus() * 4 * 4 * 64;
    switch (dt) {
      case DT_F32: return launch_strip_ks<DT_F32, 4>(a, st);
      case DT_F16: return cv8 ? launch_strip_ks<DT_F16, 8>(a, st) : launch_strip_ks<DT_F16, 4>(a, st);
      case DT_BF16: return cv8 ? launch_strip_ks<DT_BF16, 8>(a, st) : launch_strip_ks<DT_BF16, 4>(a, st);
      default: return hipErrorInvalidValue;
    }
  }
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
