// conv_pw_narrow.hip -- pointwise conv with at most 4 output channels (one
// NHWC-C4 vector per pixel): the segmentation heads (24 -> 2, 128 -> 2). A
// 128-pixel x 32-channel MFMA tile would compute 28 zero channels of every 32;
// here a group of G lanes owns one pixel: lane g reads input channel
// groups g, g + G, ... (so the group's loads cover the pixel's
// contiguous channels, one coalesced run per step), does the 4 dot products
// on the VALU against its weight vectors (read straight from memory, where
// every workgroup finds them in the caches: no LDS staging, no barrier, so
// the activation and weight loads are in flight together), and the group
// adds its partial sums by butterfly shuffles (a fixed order). It is HBM-bound: (K + 4 (+4
// res)) * storage bytes per pixel. The role of the reference's Gemv variant
// (gemm_pw.rs:91-102) and ai-cpu's pw_dot
// (crates/ai-cpu/src/kernels/pw_dot.rs:32-61); the epilogue order is
// act(acc + bias) (+ residual) as everywhere.
#include <hip/hip_runtime.h>

#include <algorithm>

#include "aih_device.h"
#include "conv_pw_narrow.h"

namespace aih {
namespace {

// Lanes per pixel G: 16 for at least 16 kg (a 128-channel head takes two
// steps of 64 channels), else 1: a lane owns a pixel and issues all of its
// loads before the first product -- KGT (4, 8 or 16, at least kg) of them,
// the ones past kg reading the last group again (cache hits, never summed),
// so the loads need no predicate: a 24-channel head reads 48 contiguous bytes
// a lane, 3 KB a wavefront in flight -- then sums them in channel order
// against the weights, which the workgroup first copies to LDS in fp32 (a
// wavefront-uniform address: broadcast reads).
template <int DTA, int DTW, int G, int KGT>
__global__ __launch_bounds__(256) void pw_narrow_kernel(PwNarrowArgs a) {
  // packed weights with one column group (NG = 1): vector (kg, j) -- input
  // channels 4kg..4kg+3 of output channel j -- at kg * 4 + j (pack.rs:95)
  const f32x4 bias = Vec4IO<DTA>::load(a.bias, 0);
  const Act ap = act_params(a.act);
  const uint32_t g = threadIdx.x % G;
  const uint32_t per_block = 256 / G;
  __shared__ f32x4 wl[G == 1 ? KGT * 4 : 1];
  if constexpr (G == 1) {
    for (uint32_t i = threadIdx.x; i < a.KG * 4; i += 256) wl[i] = narrow_w4<DTA, DTW>(a.w, i);
    __syncthreads();
  }
  for (uint32_t m0 = blockIdx.x * per_block; m0 < a.M; m0 += gridDim.x * per_block) {
    const uint32_t m = m0 + threadIdx.x / G;
    const bool pv = m < a.M;
    f32x4 acc = {};
    const size_t xrow = (size_t)(pv ? m : 0) * a.KGX;
    if constexpr (G == 1) {
      f32x4 xs[KGT];
#pragma unroll
      for (uint32_t kg = 0; kg < (uint32_t)KGT; ++kg) xs[kg] = Vec4IO<DTA>::load(a.x, xrow + min(kg, a.KG - 1));
      // every load issued before the first product (the compiler would sink
      // each load to its use behind the uniform exit below)
#pragma unroll
      for (int kg = 0; kg < KGT; ++kg) asm volatile("" : "+v"(xs[kg]));
#pragma unroll
      for (uint32_t kg = 0; kg < (uint32_t)KGT; ++kg) {
        if (kg >= a.KG) break;
        const f32x4 xv = pv ? xs[kg] : f32x4{};
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[j] += narrow_dot4(xv, wl[kg * 4 + j]);
      }
    } else {
#pragma unroll 2
      for (uint32_t kg = g; kg < a.KG; kg += G) {
        const f32x4 xl = Vec4IO<DTA>::load(a.x, xrow + kg);
        const f32x4 xv = pv ? xl : f32x4{};
        f32x4 wv[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) wv[j] = narrow_w4<DTA, DTW>(a.w, (size_t)kg * 4 + j);
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[j] += narrow_dot4(xv, wv[j]);
      }
    }
    // the group's partial sums, added by butterfly (every lane ends with the total)
#pragma unroll
    for (int off = G / 2; off > 0; off /= 2) {
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[j] += __shfl_xor(acc[j], off, G);
    }
    if (!pv || g != 0) continue;
    float v[4] = {acc.x + bias.x, acc.y + bias.y, acc.z + bias.z, acc.w + bias.w};
    act_array<4>(ap, v);
    f32x4 o = f32x4{v[0], v[1], v[2], v[3]};
    if (a.has_res) o += Vec4IO<DTA>::load(a.res, m);
    Vec4IO<DTA>::store(a.y, m, o);
  }
}

template <int DTA, int DTW, int G, int KGT>
hipError_t launch_g(const PwNarrowArgs &a, hipStream_t st) {
  const uint32_t per_block = 256 / G;
  const uint32_t blocks = (uint32_t)std::min<uint64_t>((a.M + per_block - 1) / per_block, 65535);
  hipLaunchKernelGGL((pw_narrow_kernel<DTA, DTW, G, KGT>), dim3(blocks), dim3(256), 0, st, a);
  return hipGetLastError();
}

template <int DTA, int DTW>
hipError_t launch_inst(const PwNarrowArgs &a, hipStream_t st) {
  const uint32_t g = pw_narrow_group(a.KG);
  if (g == 16) return launch_g<DTA, DTW, 16, 0>(a, st);
  if (a.KG <= 4) return launch_g<DTA, DTW, 1, 4>(a, st);
  if (a.KG <= 8) return launch_g<DTA, DTW, 1, 8>(a, st);
  return launch_g<DTA, DTW, 1, 16>(a, st);
}

}  // namespace

hipError_t launch_pw_narrow(const PwNarrowArgs &a, int dta, int dtw, hipStream_t st) {
  if (dta == DT_F32) {
    switch (dtw) {
      case DT_F32: return launch_inst<DT_F32, DT_F32>(a, st);
      case DT_F16: return launch_inst<DT_F32, DT_F16>(a, st);
      case DT_BF16: return launch_inst<DT_F32, DT_BF16>(a, st);
      default: return hipErrorInvalidValue;
    }
  }
  if (dta != dtw) return hipErrorInvalidValue;
  if (dta == DT_F16) return launch_inst<DT_F16, DT_F16>(a, st);
  if (dta == DT_BF16) return launch_inst<DT_BF16, DT_BF16>(a, st);
  return hipErrorInvalidValue;
}

}  // namespace aih
