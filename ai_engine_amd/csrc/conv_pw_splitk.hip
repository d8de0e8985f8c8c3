// conv_pw_splitk.hip -- pointwise conv GEMM for small M and long K in one
// dispatch: the skinny late layers of a segmentation encoder at batch 1
// (960 -> 160 at 10x18: 180 pixels, K = 960). The reference gives these shapes
// its in-workgroup split-K kernel (crates/ai-gpu/src/kernels/shaders/
// gemm_pw_splitk.wgsl:1-57, chosen by gemm_pw.rs:91-102): K cut across the
// threads of a workgroup and reduced on chip before the epilogue, instead of
// partial sums through memory and a second launch.
//
// Here a workgroup owns a 16-pixel x 16-channel output block and its W
// wavefronts split K: wave w runs K steps [w*spw, (w+1)*spw) on MFMA with
// its operands loaded straight from memory into registers (16-byte loads),
// then writes its 16x16 fp32 partial to LDS; after one barrier wavefront 0
// (whose bias and residual loads went out with its K operands) sums the W
// partials in wave order (a fixed order: the result does not
// depend on timing) and applies act(acc + bias) (+ residual)
// (common/epilogue.rs:13-30). 16x16 blocks rather than 32x32 give 4x more
// workgroups, so a 180-pixel layer spreads over 120 CUs instead of 30.
//
// MFMA operands (weights = A, rows = output channels; pixels = B): lane l
// supplies row / column l%16 and the K slice of its lane group q = l/16:
//   fp32  v_mfma_f32_16x16x4f32: one 16-byte load per operand holds one kg
//         (4 channels); a K step is 4 kg (kg = 4s + q) and 4 MFMAs, MFMA c
//         taking component c of both operands;
//   16-bit v_mfma_f32_16x16x32_{f16,bf16}: lane group q supplies kg 8s + 2q
//         and 8s + 2q + 1 (two 8-byte loads, 8 channels); one MFMA a step.
// Result lane l holds pixel l%16 and channels 4q .. 4q + 3 of the block: one
// NHWC-C4 vector, stored with one 16- or 8-byte store.
#include <hip/hip_runtime.h>

#include "aih_device.h"
#include "conv_pw_splitk.h"

namespace aih {
namespace {

// K steps a wavefront loads before its MFMAs (operands in flight together).
constexpr int kSplitkBatch = 4;

template <int DT, int W>
__global__ __launch_bounds__(64 * W) void pw_splitk_kernel(PwSplitkArgs a) {
  constexpr bool F32 = DT == DT_F32;
  __shared__ f32x4 part[W][64];
  const int lane = threadIdx.x & 63, q = lane >> 4, l16 = lane & 15;
  const int wave = threadIdx.x >> 6;
  const uint32_t b = xcd_remap(blockIdx.x, gridDim.x, a.nxcd);
  const uint32_t mb = b / a.nblk, nb = b - mb * a.nblk;
  const uint32_t p = mb * 16 + l16;  // this lane's pixel (B column, output pixel)
  const uint32_t n = nb * 16 + l16;  // this lane's output channel (A row)
  const bool pv = p < a.M;
  const size_t xrow = (size_t)(pv ? p : 0) * a.KG;
  const uint32_t s0 = wave * a.spw;
  const uint32_t s1 = s0 + a.spw < a.steps ? s0 + a.spw : a.steps;
  // the epilogue's operands (wavefront 0): loaded with the K operands, so the
  // launch waits on memory once, not again after the reduction
  const uint32_t c0 = nb * 16 + 4 * q;
  const size_t vi = (size_t)p * (a.N4 / 4) + c0 / 4;
  f32x4 bv = {0.0f, 0.0f, 0.0f, 0.0f}, rv = {0.0f, 0.0f, 0.0f, 0.0f};
  if (wave == 0) {
    bv = Vec4IO<DT>::load(a.bias, c0 / 4);
    if (a.has_res && pv) rv = Vec4IO<DT>::load(a.res, vi);
  }

  f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
  for (uint32_t sb = s0; sb < s1; sb += kSplitkBatch) {
    u32x4 wv[kSplitkBatch], xv[kSplitkBatch];
#pragma unroll
    for (int i = 0; i < kSplitkBatch; ++i) {
      const uint32_t s = sb + i;
      wv[i] = u32x4{0u, 0u, 0u, 0u};
      xv[i] = u32x4{0u, 0u, 0u, 0u};
      if (s >= s1) continue;
      if constexpr (F32) {
        const uint32_t kg = 4 * s + q;
        if (kg < a.KG) {
          wv[i] = reinterpret_cast<const u32x4 *>(a.w)[(size_t)kg * a.N4 + n];
          if (pv) xv[i] = reinterpret_cast<const u32x4 *>(a.x)[xrow + kg];
        }
      } else {
        const uint32_t kg = 8 * s + 2 * q;
        const u32x2 *wp = reinterpret_cast<const u32x2 *>(a.w), *xp = reinterpret_cast<const u32x2 *>(a.x);
        const u32x2 z = {0u, 0u};
        const u32x2 wlo = kg < a.KG ? wp[(size_t)kg * a.N4 + n] : z;
        const u32x2 whi = kg + 1 < a.KG ? wp[(size_t)(kg + 1) * a.N4 + n] : z;
        const u32x2 xlo = pv && kg < a.KG ? xp[xrow + kg] : z;
        const u32x2 xhi = pv && kg + 1 < a.KG ? xp[xrow + kg + 1] : z;
        wv[i] = u32x4{wlo.x, wlo.y, whi.x, whi.y};
        xv[i] = u32x4{xlo.x, xlo.y, xhi.x, xhi.y};
      }
    }
#pragma unroll
    for (int i = 0; i < kSplitkBatch; ++i) {
      if (sb + i >= s1) break;
      if constexpr (F32) {
        const f32x4 fw = __builtin_bit_cast(f32x4, wv[i]), fx = __builtin_bit_cast(f32x4, xv[i]);
#pragma unroll
        for (int c = 0; c < 4; ++c) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(fw[c], fx[c], acc, 0, 0, 0);
      } else if constexpr (DT == DT_F16) {
        acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, wv[i]),
                                                     __builtin_bit_cast(f16x8, xv[i]), acc, 0, 0, 0);
      } else {
        acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, wv[i]),
                                                      __builtin_bit_cast(bf16x8, xv[i]), acc, 0, 0, 0);
      }
    }
  }

  if constexpr (W > 1) {
    part[wave][lane] = acc;
    __syncthreads();
    if (wave != 0) return;
#pragma unroll
    for (int w = 1; w < W; ++w) acc += part[w][lane];
  }
  if (!pv) return;
  f32x4 o = acc + bv;
  o = act4(act_params(a.act), o);
  if (a.has_res) o += rv;
  Vec4IO<DT>::store(a.y, vi, o);
}

template <int DT>
hipError_t launch_dt(const PwSplitkArgs &a, uint32_t waves, hipStream_t st) {
  const dim3 grid(a.mblk * a.nblk);
  switch (waves) {
    case 1: hipLaunchKernelGGL((pw_splitk_kernel<DT, 1>), grid, dim3(64), 0, st, a); break;
    case 2: hipLaunchKernelGGL((pw_splitk_kernel<DT, 2>), grid, dim3(128), 0, st, a); break;
    case 4: hipLaunchKernelGGL((pw_splitk_kernel<DT, 4>), grid, dim3(256), 0, st, a); break;
    case 8: hipLaunchKernelGGL((pw_splitk_kernel<DT, 8>), grid, dim3(512), 0, st, a); break;
    case 16: hipLaunchKernelGGL((pw_splitk_kernel<DT, 16>), grid, dim3(1024), 0, st, a); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace

hipError_t launch_pw_splitk(const PwSplitkArgs &a, int dt, uint32_t waves, hipStream_t st) {
  if (a.N4 == 0 || a.N4 % 16 || a.N4 / 16 != a.nblk || a.mblk != (a.M + 15) / 16 || a.spw == 0 ||
      (uint64_t)a.spw * waves < a.steps)
    return hipErrorInvalidValue;
  switch (dt) {
    case DT_F32: return launch_dt<DT_F32>(a, waves, st);
    case DT_F16: return launch_dt<DT_F16>(a, waves, st);
    case DT_BF16: return launch_dt<DT_BF16>(a, waves, st);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace aih
