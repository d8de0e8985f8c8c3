// conv_stem.hip -- 3x3 conv over an image with at most 3 channels (the stem:
// 3 -> 32, stride 2, of the segmentation encoders).
//
// The generic implicit GEMM walks K in (tap, 4-channel group) units: with one
// group per tap its K of 9 groups is padded to two 32-channel stages and every
// A load is half a vector. The ai-cpu path gives this layer its own route for
// the same reason (im2row then a 1x1 GEMM, crates/ai-cpu/src/kernels/im2row.rs:22-104,
// K order (ky, kx, ic)). Here the 27 (tap, channel) values of an output pixel
// are gathered straight into the MFMA B operand -- K = tap*3 + ic, padded to
// 32 -- so one 32-pixel x 32-channel block is 2 MFMAs (f16 / bf16, K 16 each)
// or 16 MFMAs (fp32, K 2 each). A wavefront owns 32 output pixels at a time
// (grid-stride over the blocks); the 9 input pixels of a lane are 9 vector
// loads of its image row neighbourhood (cached); the weights sit in registers
// for the whole launch. The epilogue is act(acc + bias) in the MFMA layout,
// then through LDS rows (+ residual) to stores of whole pixel rows.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>

#include "aih_device.h"
#include "conv_stem.h"

namespace aih {
namespace {

// channel c (0..2) of a packed 4-channel 16-bit vector
__device__ __forceinline__ uint32_t h16(u32x2 v, int c) {
  return c == 0 ? (v.x & 0xffffu) : (c == 1 ? (v.x >> 16) : (v.y & 0xffffu));
}
__device__ __forceinline__ uint32_t pk(uint32_t lo, uint32_t hi) { return lo | (hi << 16); }

// Output staging rows: 32 pixels x 32 fp32 channels per wavefront, pitch 4
// floats wider than the row so the MFMA-layout writes spread over the banks.
constexpr uint32_t kStPitch = 36;

// F32IN: the input is the model's logical NHWC fp32 image (cin_f32 channels
// per pixel, no padding), each pixel read as one 12-byte (or narrower) load
// and rounded to the storage dtype exactly as pack_nhwc rounds it, so the
// result equals pack-then-stem bit for bit without the packed copy.
template <int DT, int NOB, bool F32IN>
__global__ __launch_bounds__(256) void conv_stem_kernel(StemArgs a) {
  constexpr bool F32 = DT == DT_F32;
  __shared__ float stg[4][32 * kStPitch];
  const int lane = threadIdx.x & 63, l32 = lane & 31, lh = lane >> 5;
  float *rows = stg[threadIdx.x >> 6];
  const uint32_t NG = a.CO / 4;

  // ---- weights of output channel row ob*32 + l32, in K order tap*3 + ic ----
  // packed element (tap, kg 0, n = o, comp = ic) at ((tap*KGP)*NG + o/4)*16 + (o%4)*4 + ic (pack.rs:95)
  auto wval = [&](uint32_t o, int k) -> uint32_t {  // raw storage bits, 0 for the K padding
    if (k >= 27) return 0u;
    const int tap = k / 3, ic = k % 3;
    const size_t idx = ((size_t)tap * a.KGP * NG + o / 4) * 16 + (o % 4) * 4 + ic;
    if constexpr (F32) return reinterpret_cast<const uint32_t *>(a.w)[idx];
    else return reinterpret_cast<const uint16_t *>(a.w)[idx];
  };
  // 16-bit: A[ob][s] holds K = s*16 + lh*8 + j; fp32: Af[ob][s] holds K = 2s + lh
  u32x4 A[NOB][2];
  float Af[F32 ? NOB : 1][16];
#pragma unroll
  for (int ob = 0; ob < NOB; ++ob) {
    const uint32_t o = ob * 32 + l32;
    if constexpr (F32) {
#pragma unroll
      for (int s = 0; s < 16; ++s) Af[ob][s] = __uint_as_float(wval(o, 2 * s + lh));
    } else {
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        const int k0 = s * 16 + lh * 8;
        A[ob][s] = u32x4{pk(wval(o, k0), wval(o, k0 + 1)), pk(wval(o, k0 + 2), wval(o, k0 + 3)),
                         pk(wval(o, k0 + 4), wval(o, k0 + 5)), pk(wval(o, k0 + 6), wval(o, k0 + 7))};
      }
    }
  }
  // bias of the lane's 16 channels per output block: groups 8q + 4lh
  f32x4 bias[NOB][4];
#pragma unroll
  for (int ob = 0; ob < NOB; ++ob)
#pragma unroll
    for (int q = 0; q < 4; ++q) bias[ob][q] = Vec4IO<DT>::load(a.bias, (ob * 32 + 8 * q + 4 * lh) / 4);
  const Act actp = act_params(a.act);
  // fp32 input: the whole image batch as one buffer (the host keeps it below 2 GiB)
  const __amdgpu_buffer_rsrc_t rs_x =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(a.x), 0, (int)a.x_bytes, 0x00020000);

  const uint32_t waves = gridDim.x * 4;
  for (uint32_t blk = blockIdx.x * 4 + (threadIdx.x >> 6); blk < a.nblocks; blk += waves) {
    const uint32_t p = blk * 32 + l32;
    const bool valid = p < a.M;
    const uint32_t pp = valid ? p : 0;
    const uint32_t img = fdiv(pp, a.fd_ohw);
    const uint32_t rem = pp - img * a.OHW;
    const uint32_t oy = fdiv(rem, a.fd_ow);
    const uint32_t ox = rem - oy * a.OW;
    const int32_t iy0 = (int32_t)(oy * a.S) - a.PT, ix0 = (int32_t)(ox * a.S) - a.PL;
    const size_t ibase = (size_t)img * a.IH * a.IW;
    // the 9 input pixels (4 channels each, the 4th is the C4 padding)
    u32x2 th[F32 ? 1 : 9];
    f32x4 tf[F32 ? 9 : 1];
#pragma unroll
    for (int t = 0; t < 9; ++t) {
      const int32_t iy = iy0 + t / 3, ix = ix0 + t % 3;
      const bool in = valid && (uint32_t)iy < a.IH && (uint32_t)ix < a.IW;
      const size_t vi = ibase + (size_t)(in ? iy : 0) * a.IW + (in ? ix : 0);
      if constexpr (F32IN) {
        f32x4 v = {};
        if (a.cin_f32 == 3) {
          // one 12-byte buffer load; taps outside the image read zeros
          typedef uint32_t u32x3 __attribute__((ext_vector_type(3)));
          const u32x3 t3 = __builtin_amdgcn_raw_buffer_load_b96(rs_x, in ? (uint32_t)vi * 12u : 0x80000000u, 0, 0);
          v = f32x4{__uint_as_float(t3.x), __uint_as_float(t3.y), __uint_as_float(t3.z), 0.0f};
        } else if (in) {
          const float *xp = reinterpret_cast<const float *>(a.x) + vi * a.cin_f32;
          v.x = xp[0];
          if (a.cin_f32 > 1) v.y = xp[1];
        }
        if constexpr (F32) tf[t] = v;
        else th[t] = pack4<DT>(v);
      } else if constexpr (F32) {
        tf[t] = in ? reinterpret_cast<const f32x4 *>(a.x)[vi] : f32x4{};
      } else {
        th[t] = in ? reinterpret_cast<const u32x2 *>(a.x)[vi] : u32x2{0u, 0u};
      }
    }
    f32x16 acc[NOB];
#pragma unroll
    for (int ob = 0; ob < NOB; ++ob) acc[ob] = f32x16{};
    if constexpr (F32) {
      // lane half lh feeds K = 2s + lh: even K for lh = 0, odd for lh = 1
#pragma unroll
      for (int s = 0; s < 16; ++s) {
        const int k = 2 * s + lh;  // lh is 0 or 1: both candidates are compile-time indices
        const int ke = 2 * s, ko = 2 * s + 1;
        const float ve = ke < 27 ? tf[ke / 3][ke % 3] : 0.0f;
        const float vo = ko < 27 ? tf[ko / 3][ko % 3] : 0.0f;
        const float b = (k & 1) ? vo : ve;
#pragma unroll
        for (int ob = 0; ob < NOB; ++ob) acc[ob] = __builtin_amdgcn_mfma_f32_32x32x2f32(Af[ob][s], b, acc[ob], 0, 0, 0);
      }
    } else {
      // K = s*16 + lh*8 + j: lane half 0 / 1 of step 0 and 1 (taps 0-2 / 2-5 / 5-7 / 8)
      auto v = [&](int k) -> uint32_t { return k < 27 ? h16(th[k / 3], k % 3) : 0u; };
      const u32x4 b0l = u32x4{pk(v(0), v(1)), pk(v(2), v(3)), pk(v(4), v(5)), pk(v(6), v(7))};
      const u32x4 b0h = u32x4{pk(v(8), v(9)), pk(v(10), v(11)), pk(v(12), v(13)), pk(v(14), v(15))};
      const u32x4 b1l = u32x4{pk(v(16), v(17)), pk(v(18), v(19)), pk(v(20), v(21)), pk(v(22), v(23))};
      const u32x4 b1h = u32x4{pk(v(24), v(25)), pk(v(26), 0u), 0u, 0u};
      const u32x4 b0 = lh ? b0h : b0l, b1 = lh ? b1h : b1l;
#pragma unroll
      for (int ob = 0; ob < NOB; ++ob) {
        if constexpr (DT == DT_F16) {
          acc[ob] = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, A[ob][0]),
                                                          __builtin_bit_cast(f16x8, b0), acc[ob], 0, 0, 0);
          acc[ob] = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, A[ob][1]),
                                                          __builtin_bit_cast(f16x8, b1), acc[ob], 0, 0, 0);
        } else {
          acc[ob] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, A[ob][0]),
                                                           __builtin_bit_cast(bf16x8, b0), acc[ob], 0, 0, 0);
          acc[ob] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, A[ob][1]),
                                                           __builtin_bit_cast(bf16x8, b1), acc[ob], 0, 0, 0);
        }
      }
    }
    // lane: pixel p, channels ob*32 + 8q + 4lh + (0..3) in acc[ob][4q..4q+3];
    // act(acc + bias) goes through the wavefront's LDS rows so each store
    // instruction writes 8 whole pixel rows of the block (contiguous)
#pragma unroll
    for (int ob = 0; ob < NOB; ++ob) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const f32x4 o = f32x4{acc[ob][4 * q], acc[ob][4 * q + 1], acc[ob][4 * q + 2], acc[ob][4 * q + 3]} + bias[ob][q];
        *reinterpret_cast<f32x4 *>(rows + l32 * kStPitch + 8 * q + 4 * lh) = act4(actp, o);
      }
      __builtin_amdgcn_wave_barrier();
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint32_t px = 8 * i + (lane >> 3), pc = 4 * (lane & 7);
        const uint32_t m = blk * 32 + px;
        f32x4 o = *reinterpret_cast<const f32x4 *>(rows + px * kStPitch + pc);
        if (m < a.M) {
          const size_t vi = (size_t)m * NG + (ob * 32 + pc) / 4;
          if (a.has_res) o += Vec4IO<DT>::load(a.res, vi);
          Vec4IO<DT>::store(a.y, vi, o);
        }
      }
      __builtin_amdgcn_wave_barrier();
    }
  }
}

// Grid-stride launch of one instantiation: as many workgroups as the CUs
// hold at once (registers and LDS), so every workgroup starts in the first
// round and they all walk the blocks in step.
template <int DT, int NOB, bool F32IN>
hipError_t launch_one(const StemArgs &a, hipStream_t st, uint32_t *grid_out) {
  // workgroups per CU, asked once per process; a failed query (no device to
  // ask) plans for eight and is not kept, so a later call asks again
  static std::atomic<int> per_cu{-1};
  int pc = per_cu.load(std::memory_order_relaxed);
  if (pc < 0) {
    int v = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&v, conv_stem_kernel<DT, NOB, F32IN>, 256, 0) == hipSuccess &&
        v >= 1) {
      per_cu.store(v, std::memory_order_relaxed);
      pc = v;
    } else {
      pc = 8;
    }
  }
  const uint32_t wgs = (uint32_t)std::min<uint64_t>((a.nblocks + 3) / 4, (uint64_t)device_cus() * pc);
  if (grid_out) {
    *grid_out = wgs;
    return hipSuccess;
  }
  hipLaunchKernelGGL((conv_stem_kernel<DT, NOB, F32IN>), dim3(wgs), dim3(256), 0, st, a);
  return hipGetLastError();
}

template <int DT, int NOB>
hipError_t launch_inst(const StemArgs &a, hipStream_t st, uint32_t *grid_out) {
  return a.cin_f32 ? launch_one<DT, NOB, true>(a, st, grid_out) : launch_one<DT, NOB, false>(a, st, grid_out);
}

template <int DT>
hipError_t launch_dt(const StemArgs &a, hipStream_t st, uint32_t *grid_out) {
  switch (a.CO / 32) {
    case 1: return launch_inst<DT, 1>(a, st, grid_out);
    case 2: return launch_inst<DT, 2>(a, st, grid_out);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace

hipError_t launch_conv_stem(const StemArgs &a, int dt, hipStream_t st, uint32_t *grid_out) {
  if (a.cin_f32 > 3) return hipErrorInvalidValue;
  switch (dt) {
    case DT_F32: return launch_dt<DT_F32>(a, st, grid_out);
    case DT_F16: return launch_dt<DT_F16>(a, st, grid_out);
    case DT_BF16: return launch_dt<DT_BF16>(a, st, grid_out);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace aih
