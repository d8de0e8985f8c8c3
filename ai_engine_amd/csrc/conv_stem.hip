// conv_stem.hip -- 3x3 conv over an image with at most 3 channels (the stem:
// 3 -> 32, stride 2, of the segmentation encoders).
//
// The generic implicit GEMM walks K in (tap, 4-channel group) units: with one
// group per tap its K of 9 groups is padded to two 32-channel stages and every
// A load is half a vector. The ai-cpu path gives this layer its own route for
// the same reason (im2row then a 1x1 GEMM, crates/ai-cpu/src/kernels/im2row.rs:22-104,
// K order (ky, kx, ic)). Here the (tap, channel) values of an output pixel
// are gathered straight into the MFMA B operand: fp32 K = tap*3 + ic, padded
// to 32, 16 MFMAs (K 2 each) per 32-pixel x 32-channel block; 16-bit 4 K per
// tap (the 4th channel zero), the two lane halves holding different taps, 3
// MFMAs (K 16 each) per block and 5 input loads per lane instead of 9. The
// weights sit in registers for the whole launch. The epilogue is
// act(acc + bias) in the MFMA layout (16-bit: the bias is the MFMAs' first
// accumulator), then through LDS rows (+ residual) to stores of whole pixel
// rows.
//
// Every wavefront walks a contiguous run of 32-pixel blocks, the next two
// blocks' input pixels in flight while the current one computes;
// consecutive runs go to the workgroups of one XCD (xcd_remap), so the input
// row that vertically adjacent output rows share (stride 2: every other row)
// is read from HBM once and found in that XCD's L2 the second time. (With
// blocks dealt round-robin over the grid, the two readers of a shared row
// sat on different XCDs: 1.55x the input read from HBM.)
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <type_traits>

#include "aih_device.h"
#include "conv_stem.h"

namespace aih {
namespace {

// Output staging rows: 32 pixels x 32 fp32 channels per wavefront, pitch 4
// floats wider than the row so the MFMA-layout writes spread over the banks.
constexpr uint32_t kStPitch = 36;

// FIN: the input's form. 0: NHWC-C4 in the storage dtype. 3 / 1: the model's
// logical NHWC fp32 image (cin_f32 channels per pixel, no padding) -- 3
// channels as one 12-byte buffer load per pixel, 1 or 2 channels as one
// 4-byte buffer load per channel -- rounded to the storage dtype exactly as
// pack_nhwc rounds it, so the result equals pack-then-stem bit for bit
// without the packed copy. Every tap of every block issues the same loads
// (taps outside the image or past the wavefront's run read zeros), so the
// loads of the blocks in flight are never waited on early.
//
// CL: the activation is clamp-type (identity, ReLU, ReLU6, clamp01), one
// v_med3 per value with no branch; otherwise the general activation code.
template <int DT, int NOB, int FIN, bool CL>
__global__ __launch_bounds__(256) void conv_stem_kernel(StemArgs a) {
  constexpr bool F32 = DT == DT_F32;
  __shared__ float stg[4][32 * kStPitch];
  const int lane = threadIdx.x & 63, l32 = lane & 31, lh = lane >> 5;
  float *rows = stg[threadIdx.x >> 6];
  const uint32_t NG = a.CO / 4;

  // ---- weights of output channel row ob*32 + l32 ----
  // packed element (tap, kg 0, n = o, comp = ic) at ((tap*KGP)*NG + o/4)*16 + (o%4)*4 + ic (pack.rs:95)
  auto wtap = [&](uint32_t o, int tap, int ic) -> uint32_t {  // raw storage bits, 0 for the K padding
    if (tap >= 9 || ic >= 3) return 0u;
    const size_t idx = ((size_t)tap * a.KGP * NG + o / 4) * 16 + (o % 4) * 4 + ic;
    if constexpr (F32) return reinterpret_cast<const uint32_t *>(a.w)[idx];
    else return reinterpret_cast<const uint16_t *>(a.w)[idx];
  };
  // 16-bit: 3 steps of K 16 (stem_a16); fp32: K = tap*3 + ic (27, padded to
  // 32), Af[ob][s] holding K = 2s + lh.
  u32x4 A[F32 ? 1 : NOB][3];
  float Af[F32 ? NOB : 1][16];
#pragma unroll
  for (int ob = 0; ob < NOB; ++ob) {
    const uint32_t o = ob * 32 + l32;
    if constexpr (F32) {
#pragma unroll
      for (int s = 0; s < 16; ++s) {
        const int k = 2 * s + lh;
        Af[ob][s] = __uint_as_float(k < 27 ? wtap(o, k / 3, k % 3) : 0u);
      }
    } else {
#pragma unroll
      for (int s = 0; s < 3; ++s) A[ob][s] = stem_a16(a.w, a.KGP, NG, o, lh, s);
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

  // The input pixels a lane loads per output pixel. fp32: all 9 taps (each
  // lane half feeds every tap). 16-bit: 5 slots, slot i holding tap
  // stem_slot_tap(lh, i), so the two halves split the loads and each slot
  // pair is one B operand.
  constexpr int NT = F32 ? 9 : 5;
  int32_t tdy[NT], tdx[NT], toff[NT];
  bool tok[NT];
#pragma unroll
  for (int i = 0; i < NT; ++i) {
    const int t0 = F32 ? i : stem_slot_tap(0, i), t1 = F32 ? i : stem_slot_tap(1, i);
    tdy[i] = lh ? t1 / 3 : t0 / 3;
    tdx[i] = lh ? t1 % 3 : t0 % 3;
    tok[i] = lh ? t1 < 9 : t0 < 9;
    toff[i] = tdy[i] * (int32_t)a.IW + tdx[i];
  }

  // this wavefront's contiguous run of blocks
  const uint32_t gw = xcd_remap(blockIdx.x, gridDim.x, a.nxcd) * 4 + (threadIdx.x >> 6), nw = gridDim.x * 4;
  // (wave-uniform: held in scalar registers, the loop's branches scalar)
  const uint32_t blk_begin = __builtin_amdgcn_readfirstlane((uint32_t)((uint64_t)gw * a.nblocks / nw));
  const uint32_t blk_end = __builtin_amdgcn_readfirstlane((uint32_t)((uint64_t)(gw + 1) * a.nblocks / nw));
  // the lane's input pixels for block blk, as loaded (fp32 input: 12 bytes;
  // fp32 NHWC-C4: 16; 16-bit NHWC-C4: 8)
  typedef uint32_t u32x3 __attribute__((ext_vector_type(3)));
  constexpr bool F32IN = FIN != 0;
  using Raw = std::conditional_t<F32IN, u32x3, std::conditional_t<F32, f32x4, u32x2>>;
  auto load_taps = [&](uint32_t blk, Raw (&raw)[NT]) {
    const uint32_t p = blk * 32 + l32;
    const bool valid = blk < blk_end && p < a.M;
    const uint32_t pp = valid ? p : 0;
    // valid as an offset bias the compiler cannot see through: a block past
    // the run issues the same loads (at offsets past the buffer, or pixel 0)
    // instead of a branch around them
    uint32_t oob = valid ? 0u : 0x80000000u;
    asm volatile("" : "+v"(oob));
    const uint32_t img = fdiv(pp, a.fd_ohw);
    const uint32_t rem = pp - img * a.OHW;
    const uint32_t oy = fdiv(rem, a.fd_ow);
    const uint32_t ox = rem - oy * a.OW;
    const int32_t iy0 = (int32_t)(oy * a.S) - a.PT, ix0 = (int32_t)(ox * a.S) - a.PL;
    // pixel index of tap (0, 0), which may lie outside the image
    const int64_t v0 = ((int64_t)img * a.IH + iy0) * a.IW + ix0;
#pragma unroll
    for (int i = 0; i < NT; ++i) {
      const int32_t iy = iy0 + tdy[i], ix = ix0 + tdx[i];
      const bool in = tok[i] && (uint32_t)iy < a.IH && (uint32_t)ix < a.IW;
      if constexpr (F32IN) {
        // below 2 GiB of input: the in-image pixel index fits 32 bits
        // (an offset at or past the buffer's size reads zeros)
        const uint32_t vi = (uint32_t)v0 + (uint32_t)toff[i];
        if constexpr (FIN == 3) {
          raw[i] = __builtin_amdgcn_raw_buffer_load_b96(rs_x, (in ? vi * 12u : 0x80000000u) | oob, 0, 0);
        } else {
          const uint32_t o = vi * a.cin_f32 * 4u;
          raw[i] = u32x3{__builtin_amdgcn_raw_buffer_load_b32(rs_x, (in ? o : 0x80000000u) | oob, 0, 0),
                         __builtin_amdgcn_raw_buffer_load_b32(rs_x, (in && a.cin_f32 > 1 ? o + 4u : 0x80000000u) | oob, 0, 0),
                         0u};
        }
      } else {
        // pixel 0 stands in for taps outside the image; the select zeroes them
        const bool use = in && oob == 0u;
        const size_t vi = use ? (size_t)(v0 + toff[i]) : 0;
        if constexpr (F32) {
          const f32x4 v = reinterpret_cast<const f32x4 *>(a.x)[vi];
          raw[i] = use ? v : f32x4{};
        } else {
          const u32x2 v = reinterpret_cast<const u32x2 *>(a.x)[vi];
          raw[i] = use ? v : u32x2{0u, 0u};
        }
      }
    }
  };

  // Block blk: its loads (issued two blocks earlier) converted out of buf,
  // buf refilled with block blk + 2's (into the same registers: nothing
  // waits on them until their own turn), then the MFMAs and the epilogue.
  // A block past the run (the odd one out of the last pair) computes on
  // zeros and stores nothing.
  auto step = [&](uint32_t blk, Raw (&raw)[NT]) {
    // 16-bit: th[i] = the slot's 4 channels (the 4th zero); fp32: tf[tap]
    u32x2 th[F32 ? 1 : NT + 1];
    f32x4 tf[F32 ? NT : 1];
#pragma unroll
    for (int i = 0; i < NT; ++i) {
      if constexpr (F32IN) {
        const f32x4 v = f32x4{__uint_as_float(raw[i].x), __uint_as_float(raw[i].y), __uint_as_float(raw[i].z), 0.0f};
        if constexpr (F32) tf[i] = v;
        else th[i] = pack4<DT>(v);
      } else if constexpr (F32) {
        tf[i] = raw[i];
      } else {
        th[i] = u32x2{raw[i].x, raw[i].y & 0xffffu};  // the 4th channel is storage padding
      }
    }
    if constexpr (!F32) th[NT] = u32x2{0u, 0u};
    // the conversion completes before the refill is issued, so the refill
    // can reuse raw's registers (loop-carried without copies)
#pragma unroll
    for (int i = 0; i < NT; ++i) {
      if constexpr (F32) asm volatile("" : "+v"(tf[i])::"memory");
      else asm volatile("" : "+v"(th[i])::"memory");
    }
    load_taps(blk + 2, raw);
    // 16-bit: the bias is the MFMAs' first accumulator (as in the stem fused
    // into the block after it, ir_wave_impl.h); fp32: added after the sum
    f32x16 acc[NOB];
#pragma unroll
    for (int ob = 0; ob < NOB; ++ob) {
      if constexpr (F32)
        acc[ob] = f32x16{};
      else
        acc[ob] = stem_acc_init(bias[ob]);
    }
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
      // step s: the lane's slots 2s and 2s + 1 (K = s*16 + lh*8 + j)
#pragma unroll
      for (int s = 0; s < 3; ++s) {
        const u32x4 b = u32x4{th[2 * s].x, th[2 * s].y, th[2 * s + 1].x, th[2 * s + 1].y};
#pragma unroll
        for (int ob = 0; ob < NOB; ++ob) {
          if constexpr (DT == DT_F16)
            acc[ob] = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, A[ob][s]),
                                                            __builtin_bit_cast(f16x8, b), acc[ob], 0, 0, 0);
          else
            acc[ob] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, A[ob][s]),
                                                             __builtin_bit_cast(bf16x8, b), acc[ob], 0, 0, 0);
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
        f32x4 o = f32x4{acc[ob][4 * q], acc[ob][4 * q + 1], acc[ob][4 * q + 2], acc[ob][4 * q + 3]};
        if constexpr (F32) o += bias[ob][q];
        f32x4 r;
        if constexpr (CL)
          r = f32x4{act_clamp_any(actp, o.x), act_clamp_any(actp, o.y), act_clamp_any(actp, o.z), act_clamp_any(actp, o.w)};
        else
          r = act4(actp, o);
        *reinterpret_cast<f32x4 *>(rows + l32 * kStPitch + 8 * q + 4 * lh) = r;
      }
      __builtin_amdgcn_wave_barrier();
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint32_t px = 8 * i + (lane >> 3), pc = 4 * (lane & 7);
        const uint32_t m = blk * 32 + px;
        f32x4 o = *reinterpret_cast<const f32x4 *>(rows + px * kStPitch + pc);
        if (blk < blk_end && m < a.M) {
          const size_t vi = (size_t)m * NG + (ob * 32 + pc) / 4;
          if (a.has_res) o += Vec4IO<DT>::load(a.res, vi);
          Vec4IO<DT>::store(a.y, vi, o);
        }
      }
      __builtin_amdgcn_wave_barrier();
    }
  };
  // two buffers alternate, so two blocks' loads are in flight ahead of the
  // one being computed (no register copies that would wait on them)
  Raw bx[NT], by[NT];
  load_taps(blk_begin, bx);
  load_taps(blk_begin + 1, by);
  for (uint32_t blk = blk_begin; blk < blk_end; blk += 2) {
    step(blk, bx);
    step(blk + 1, by);
  }
}

// Grid-stride launch of one instantiation: as many workgroups as the CUs
// hold at once (registers and LDS), so every workgroup starts in the first
// round and they all walk the blocks in step.
template <int DT, int NOB, int FIN, bool CL>
hipError_t launch_one(const StemArgs &a, hipStream_t st, uint32_t *grid_out) {
  // workgroups per CU, asked once per process; a failed query (no device to
  // ask) plans for eight and is not kept, so a later call asks again
  static std::atomic<int> per_cu{-1};
  int pc = per_cu.load(std::memory_order_relaxed);
  if (pc < 0) {
    int v = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&v, conv_stem_kernel<DT, NOB, FIN, CL>, 256, 0) == hipSuccess &&
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
  hipLaunchKernelGGL((conv_stem_kernel<DT, NOB, FIN, CL>), dim3(wgs), dim3(256), 0, st, a);
  return hipGetLastError();
}

template <int DT, int NOB>
hipError_t launch_inst(const StemArgs &a, hipStream_t st, uint32_t *grid_out) {
  if (act_is_clamp(a.act)) {
    if (a.cin_f32 == 3) return launch_one<DT, NOB, 3, true>(a, st, grid_out);
    return a.cin_f32 ? launch_one<DT, NOB, 1, true>(a, st, grid_out) : launch_one<DT, NOB, 0, true>(a, st, grid_out);
  }
  if (a.cin_f32 == 3) return launch_one<DT, NOB, 3, false>(a, st, grid_out);
  return a.cin_f32 ? launch_one<DT, NOB, 1, false>(a, st, grid_out) : launch_one<DT, NOB, 0, false>(a, st, grid_out);
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
