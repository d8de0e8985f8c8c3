// conv_pw_narrow.hip -- pointwise conv with at most 4 output channels (one
// NHWC-C4 vector per pixel): the segmentation heads (24 -> 2, 128 -> 2). A
// 128-pixel x 32-channel MFMA tile would compute 28 zero channels of every 32;
// here one thread owns one pixel, reads its K channels once (16-byte loads),
// and does the 4 dot products on the VALU against weights staged in LDS. It
// is HBM-bound: (K + 4 (+4 res)) * storage bytes per pixel. The role of the
// reference's Gemv variant (gemm_pw.rs:91-102) and ai-cpu's pw_dot
// (crates/ai-cpu/src/kernels/pw_dot.rs:32-61); the epilogue order is
// act(acc + bias) (+ residual) as everywhere.
#include <hip/hip_runtime.h>

#include <algorithm>

#include "aih_device.h"
#include "conv_pw_narrow.h"

namespace aih {
namespace {

template <int DTA, int DTW>
__device__ __forceinline__ f32x4 ld_w4(const void *w, size_t vi) {
  if constexpr (DTW == DT_F32) return reinterpret_cast<const f32x4 *>(w)[vi];
  else return unpack4<DTW>(reinterpret_cast<const u32x2 *>(w)[vi]);
}

template <int DTA, int DTW>
__global__ __launch_bounds__(256) void pw_narrow_kernel(PwNarrowArgs a) {
  extern __shared__ f32x4 wl[];  // [KG][4]: input channels 4kg..4kg+3 of output channel j
  // packed weights with one column group (NG = 1): vector (kg, j) at kg * 4 + j (pack.rs:95)
  for (uint32_t i = threadIdx.x; i < a.KG * 4; i += 256) wl[i] = ld_w4<DTA, DTW>(a.w, i);
  __syncthreads();
  const f32x4 bias = Vec4IO<DTA>::load(a.bias, 0);
  const Act ap = act_params(a.act);
  for (uint32_t m = blockIdx.x * 256 + threadIdx.x; m < a.M; m += gridDim.x * 256) {
    f32x4 acc = {};
    const size_t xrow = (size_t)m * a.KGX;
    for (uint32_t kg = 0; kg < a.KG; ++kg) {
      const f32x4 xv = Vec4IO<DTA>::load(a.x, xrow + kg);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const f32x4 wv = wl[kg * 4 + j];
        acc[j] += xv.x * wv.x + xv.y * wv.y + xv.z * wv.z + xv.w * wv.w;
      }
    }
    float v[4] = {acc.x + bias.x, acc.y + bias.y, acc.z + bias.z, acc.w + bias.w};
    act_array<4>(ap, v);
    f32x4 o = f32x4{v[0], v[1], v[2], v[3]};
    if (a.has_res) o += Vec4IO<DTA>::load(a.res, m);
    Vec4IO<DTA>::store(a.y, m, o);
  }
}

template <int DTA, int DTW>
hipError_t launch_inst(const PwNarrowArgs &a, hipStream_t st) {
  const uint32_t blocks = (uint32_t)std::min<uint64_t>((a.M + 255) / 256, 4096);
  hipLaunchKernelGGL((pw_narrow_kernel<DTA, DTW>), dim3(blocks), dim3(256), a.KG * 4 * sizeof(f32x4), st, a);
  return hipGetLastError();
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
