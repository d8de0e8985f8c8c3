// conv_pw_direct.hip -- pointwise conv with short K (<= 128 16-bit / 64 fp32
// channels) and at most 64 output channels: the thin 1x1 layers of the
// segmentation models (44 -> 24, 32 -> 12, 96 -> 48, 32 -> 64). The tiled
// GEMM stages K through LDS in 16/32-channel steps behind barriers; with one
// or two steps per tile its global-load latency is exposed on every tile.
// Here a wavefront owns 32 output pixels at a time (grid-stride), loads the
// whole K of its pixels and of the weights straight into MFMA operand
// registers (16-byte loads; the weights are shared by every wavefront and
// come from the caches), and runs the K steps back to back for each 32-channel
// block of the output. Same MFMA operand convention as the GEMM: weights are
// A (rows = output channels), the 32 pixels are B; lane l of the result holds
// pixel l%32 and channels 8*(r/4) + 4*(l/32) + r%4. The epilogue is
// act(acc + bias) (+ residual) (common/epilogue.rs:13-30), stored as one
// 4-channel vector per lane and group. The route of gemm_pw.rs:91-102's small
// tiles for these shapes.
#include <hip/hip_runtime.h>

#include <algorithm>

#include "aih_device.h"
#include "conv_pw_direct.h"

namespace aih {
namespace {

// KS: K steps of one MFMA operand (16-bit: 16 channels = 4 kg per step;
// fp32: 8 channels = 2 kg per step, four v_mfma_f32_32x32x2f32 each).
// WPG: wavefronts per workgroup; the wavefronts share nothing, so a launch
// with fewer 32-pixel blocks than four per CU takes one-wavefront
// workgroups, which the dispatcher spreads over every CU.
template <int DT, int KS, int NOB, int WPG>
__global__ __launch_bounds__(64 * WPG) void pw_direct_kernel(PwDirectArgs a) {
  constexpr bool F32 = DT == DT_F32;
  const int lane = threadIdx.x & 63, l32 = lane & 31, lh = lane >> 5;
  const Act actp = act_params(a.act);
  const uint32_t ks_used = F32 ? (a.KG + 1) / 2 : (a.KG + 3) / 4;

  // lane's weight operands for every K step and output block (K slice as the
  // activations): f32 -> kg = 2s + lh, 16 bytes; 16-bit -> kg = 4s + 2lh and
  // 4s + 2lh + 1, 8 bytes each (columns N4 apart in the packed layout)
  u32x4 wop[NOB][KS];
#pragma unroll
  for (int ob = 0; ob < NOB; ++ob) {
    const uint32_t n = ob * 32 + l32;
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      u32x4 v = {0u, 0u, 0u, 0u};
      if constexpr (F32) {
        const uint32_t kg = 2 * s + lh;
        if (s < (int)ks_used && kg < a.KG && n < a.N4) v = reinterpret_cast<const u32x4 *>(a.w)[(size_t)kg * a.N4 + n];
      } else {
        const uint32_t kg = 4 * s + 2 * lh;
        if (s < (int)ks_used && n < a.N4) {
          const u32x2 *wp = reinterpret_cast<const u32x2 *>(a.w);
          const u32x2 lo = kg < a.KG ? wp[(size_t)kg * a.N4 + n] : u32x2{0u, 0u};
          const u32x2 hi = kg + 1 < a.KG ? wp[(size_t)(kg + 1) * a.N4 + n] : u32x2{0u, 0u};
          v = u32x4{lo.x, lo.y, hi.x, hi.y};
        }
      }
      wop[ob][s] = v;
    }
  }
  // bias of the lane's 16 channels per block: groups 8q + 4lh
  f32x4 bias[NOB][4];
#pragma unroll
  for (int ob = 0; ob < NOB; ++ob)
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const uint32_t c = ob * 32 + 8 * q + 4 * lh;
      bias[ob][q] = c < a.N4 ? Vec4IO<DT>::load(a.bias, c / 4) : f32x4{};
    }

  const uint32_t waves = gridDim.x * WPG;
  for (uint32_t blk = blockIdx.x * WPG + (threadIdx.x >> 6); blk < a.nblk; blk += waves) {
    const uint32_t p = blk * 32 + l32;
    const bool valid = p < a.M;
    const size_t xrow = (size_t)(valid ? p : 0) * a.KG;
    u32x4 xop[KS];
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      u32x4 v = {0u, 0u, 0u, 0u};
      if constexpr (F32) {
        const uint32_t kg = 2 * s + lh;
        if (s < (int)ks_used && kg < a.KG) v = reinterpret_cast<const u32x4 *>(a.x)[xrow + kg];
      } else {
        const uint32_t kg = 4 * s + 2 * lh;
        if (s < (int)ks_used) {
          const u32x2 *xp = reinterpret_cast<const u32x2 *>(a.x);
          const u32x2 lo = kg < a.KG ? xp[xrow + kg] : u32x2{0u, 0u};
          const u32x2 hi = kg + 1 < a.KG ? xp[xrow + kg + 1] : u32x2{0u, 0u};
          v = u32x4{lo.x, lo.y, hi.x, hi.y};
        }
      }
      xop[s] = v;
    }
#pragma unroll
    for (int ob = 0; ob < NOB; ++ob) {
      f32x16 acc = {};
#pragma unroll
      for (int s = 0; s < KS; ++s) {
        if (s >= (int)ks_used) break;
        if constexpr (F32) {
          const f32x4 wv = __builtin_bit_cast(f32x4, wop[ob][s]), xv = __builtin_bit_cast(f32x4, xop[s]);
#pragma unroll
          for (int c = 0; c < 4; ++c) acc = __builtin_amdgcn_mfma_f32_32x32x2f32(wv[c], xv[c], acc, 0, 0, 0);
        } else if constexpr (DT == DT_F16) {
          acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, wop[ob][s]),
                                                      __builtin_bit_cast(f16x8, xop[s]), acc, 0, 0, 0);
        } else {
          acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, wop[ob][s]),
                                                       __builtin_bit_cast(bf16x8, xop[s]), acc, 0, 0, 0);
        }
      }
      if (!valid) continue;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const uint32_t c = ob * 32 + 8 * q + 4 * lh;
        if (c >= a.N4) continue;
        f32x4 o = f32x4{acc[4 * q], acc[4 * q + 1], acc[4 * q + 2], acc[4 * q + 3]} + bias[ob][q];
        o = act4(actp, o);
        const size_t vi = (size_t)p * (a.N4 / 4) + c / 4;
        if (a.has_res) o += Vec4IO<DT>::load(a.res, vi);
        Vec4IO<DT>::store(a.y, vi, o);
      }
    }
  }
}

// Launch (or, with grid_out, only size) one instantiation. Small launches
// take one wavefront per block; larger ones are grid-stride with 4
// wavefronts per workgroup and as many workgroups as the CUs hold at once
// (the instantiation's occupancy), so none waits for a second round.
template <int DT, int KS, int NOB>
hipError_t launch_inst(const PwDirectArgs &a, hipStream_t st, uint32_t *grid_out) {
  const uint32_t cus = device_cus();
  const bool one = pw_direct_waves_per_group(a.nblk, cus) == 1;
  uint32_t grid = a.nblk;
  if (!one) {
    static int per_cu = -1;
    if (per_cu < 0) {
      int v = 0;
      if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&v, pw_direct_kernel<DT, KS, NOB, 4>, 256, 0) != hipSuccess ||
          v < 1)
        v = 8;  // no device to ask: eight workgroups per CU
      per_cu = v;
    }
    const uint64_t wgs = ((uint64_t)a.nblk + 3) / 4, cap = (uint64_t)cus * per_cu;
    grid = (uint32_t)(wgs < cap ? wgs : cap);
  }
  if (grid_out) {
    *grid_out = grid;
    return hipSuccess;
  }
  if (one)
    hipLaunchKernelGGL((pw_direct_kernel<DT, KS, NOB, 1>), dim3(grid), dim3(64), 0, st, a);
  else
    hipLaunchKernelGGL((pw_direct_kernel<DT, KS, NOB, 4>), dim3(grid), dim3(256), 0, st, a);
  return hipGetLastError();
}

template <int DT, int KS>
hipError_t launch_ks(const PwDirectArgs &a, hipStream_t st, uint32_t *grid_out) {
  return a.N4 <= 32 ? launch_inst<DT, KS, 1>(a, st, grid_out) : launch_inst<DT, KS, 2>(a, st, grid_out);
}

template <int DT>
hipError_t launch_dt(const PwDirectArgs &a, hipStream_t st, uint32_t *grid_out) {
  // K steps: fp32 8 channels, 16-bit 16 channels
  const uint32_t ks = DT == DT_F32 ? (a.KG + 1) / 2 : (a.KG + 3) / 4;
  if (ks <= 2) return launch_ks<DT, 2>(a, st, grid_out);
  if (ks <= 4) return launch_ks<DT, 4>(a, st, grid_out);
  if (ks <= 8) return launch_ks<DT, 8>(a, st, grid_out);
  return hipErrorInvalidValue;
}

}  // namespace

hipError_t launch_pw_direct(const PwDirectArgs &a, int dt, hipStream_t st, uint32_t *grid_out) {
  if (a.N4 > kPwDirectMaxN4 || a.N4 % 4) return hipErrorInvalidValue;
  switch (dt) {
    case DT_F32: return launch_dt<DT_F32>(a, st, grid_out);
    case DT_F16: return launch_dt<DT_F16>(a, st, grid_out);
    case DT_BF16: return launch_dt<DT_BF16>(a, st, grid_out);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace aih
