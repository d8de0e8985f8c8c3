// conv_igemm_direct.hip -- 3x3 implicit-GEMM conv with at most 64 output
// channels (and, as a one-tap launch, pointwise convs with mid-size K), the
// weights resident in LDS and the activations loaded straight into MFMA
// operand registers.
//
// The tiled GEMM stages A and B through LDS in 16/32-channel steps behind a
// workgroup barrier each; with 32 or 64 output columns a step holds only 2-8
// MFMAs per wavefront, so the barrier and the staging round trip set the pace
// (a 72 -> 32 3x3 conv at 40x72 batch 64 ran at 7 % of both rooflines).
// Here the workgroup copies the whole packed weight tensor (9 taps x K x N)
// into LDS once, reordered into MFMA A operands, and then never synchronises
// again: each of its eight wavefronts owns 32 output pixels at a time, decodes
// their source pixels per tap in registers (implicit im2col, no buffer) and
// loads the tap's input channels as 16-byte buffer loads straight into MFMA B
// operands -- out-of-image taps and padding units read zeros from the buffer
// range check. Loads run a ring of D steps ahead of the MFMAs, across block
// ends. The reference's route for the same layers is
// conv_igemm_{tiled,direct}.wgsl (crates/ai-gpu/src/kernels/conv_igemm.rs);
// for the pointwise launches (TAPS = 1, the pixel row as the image, up to 256
// fp32 outputs as column groups of 64 that are separate work items) it is
// gemm_pw_tiled.wgsl (crates/ai-gpu/src/kernels/gemm_pw.rs).
//
// K order: tap-major (ky, kx), then the input parts in order, then 16-byte
// units of each part; MFMA step j of a tap pairs unit 2j (lane half 0) with
// unit 2j + 1 (lane half 1) of one part, the same pairing for both operands.
// A 16-byte unit is 4 fp32 channels (one kg: four v_mfma_f32_32x32x2f32, one
// per component) or 8 16-bit channels (two kg: one v_mfma_f32_32x32x16).
// Lane l of the result holds pixel l%32 and channels 8*(r/4) + 4*(l/32) + r%4;
// the epilogue is act(acc + bias) (+ residual) (common/epilogue.rs:13-30),
// one 4-channel vector per lane and group.
#include <hip/hip_runtime.h>

#include <algorithm>

#include "conv_igemm_direct.h"

namespace aih {
namespace {

constexpr uint32_t kOob = 0x80000000u;  // a byte offset past every part's buffer
constexpr int kWaves = kIgDirectThreads / 64;
// Output staging rows: 32 pixels x 32 fp32 channels per wavefront, the row
// pitch 4 floats wider so the MFMA-layout writes (8 pixels, one 16-byte piece
// each, per LDS cycle) fall in distinct banks.
constexpr uint32_t kStPitch = 36;
constexpr uint32_t kStBytes = kWaves * 32 * kStPitch * 4;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t ig_rsrc(const void *base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), 0, (int)bytes, 0x00020000);
}

template <int DT, int NOB, int TAPS, int NJ, int D>
__global__ __launch_bounds__(kIgDirectThreads) void conv_igemm_direct_kernel(IgDirectArgs a) {
  constexpr bool F32 = DT == DT_F32;
  constexpr int NC = NOB * 32;  // weight columns in LDS
  extern __shared__ __align__(16) char lds[];
  u32x4 *Wl = reinterpret_cast<u32x4 *>(lds);
  const uint32_t nj0 = a.nj0;
  // LDS row of one (tap, step, half): every column group's NC columns
  const uint32_t RS = a.ncg * NC;
  float *Bl = reinterpret_cast<float *>(lds + TAPS * NJ * 2 * RS * 16);

  const int tid = threadIdx.x, lane = tid & 63, l32 = lane & 31, lh = lane >> 5;
  // the wavefront index in a scalar register: block indices and the loop's
  // exit test stay uniform (scalar branches, no exec-mask regions)
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);

  // ---- weights -> LDS as [tap][step][half][column] operands (zero padding) ----
  // each thread issues a batch of loads before the batch's LDS stores, so the
  // copy costs one memory latency per batch (one batch up to 4096 entries)
  const uint32_t nw = TAPS * NJ * 2 * RS;
  constexpr int BATCH = 8;
  for (uint32_t base = 0; base < nw; base += BATCH * kIgDirectThreads) {
    u32x4 wst[BATCH];
#pragma unroll
    for (int k = 0; k < BATCH; ++k) {
      const uint32_t i = base + tid + k * kIgDirectThreads;
      const uint32_t n = i % RS, r = i / RS, h = r & 1, r2 = r >> 1, j = r2 % NJ, tap = r2 / NJ;
      const uint32_t p = j >= nj0 ? 1 : 0;
      const uint32_t u = 2 * (j - (p ? nj0 : 0)) + h;
      u32x4 v = {0u, 0u, 0u, 0u};
      if (i < nw && u < a.nu[p] && n < a.N4) {
        if constexpr (F32) {
          const uint32_t kg = a.kg_first[p] + u;
          v = reinterpret_cast<const u32x4 *>(a.w)[(size_t)(tap * a.KGP + kg) * a.N4 + n];
        } else {
          const uint32_t kg = a.kg_first[p] + 2 * u;
          const u32x2 *wp = reinterpret_cast<const u32x2 *>(a.w);
          const u32x2 lo = wp[(size_t)(tap * a.KGP + kg) * a.N4 + n];
          const u32x2 hi = wp[(size_t)(tap * a.KGP + kg + 1) * a.N4 + n];
          v = u32x4{lo.x, lo.y, hi.x, hi.y};
        }
      }
      wst[k] = v;
    }
#pragma unroll
    for (int k = 0; k < BATCH; ++k) {
      const uint32_t i = base + tid + k * kIgDirectThreads;
      if (i < nw) Wl[i] = wst[k];
    }
  }
  if ((uint32_t)tid < RS) Bl[tid] = (uint32_t)tid < a.N4 ? Vec4IO<DT>::load(a.bias, tid / 4)[tid % 4] : 0.0f;
  __syncthreads();

  const __amdgpu_buffer_rsrc_t rs0 = ig_rsrc(a.src[0], a.src_bytes[0]);
  const __amdgpu_buffer_rsrc_t rs1 = ig_rsrc(a.src[1], a.src_bytes[1]);
  const Act actp = act_params(a.act);

  // this workgroup's contiguous range of work items -- item = block * ncg +
  // column group, so the column groups of one block run back to back and
  // re-read its activations from the cache (ranges go out XCD by XCD so
  // neighbouring blocks, which share input rows, meet in one L2)
  const uint32_t nitems = a.nblk * a.ncg;
  const uint32_t g = xcd_remap(blockIdx.x, gridDim.x, a.nxcd);
  const uint32_t b_begin = (uint32_t)(((uint64_t)g * nitems) / gridDim.x);
  const uint32_t b_end = (uint32_t)(((uint64_t)(g + 1) * nitems) / gridDim.x);

  // lane's weight operand of (tap, step, column group cg, block o) at
  // Wl[wl + cg*NC + (tap*NJ + step)*2*RS + o*32]
  const uint32_t wl = lh * RS + l32;

  // a block's output pixels decoded: lane pixel, the unit index (per part)
  // of its tap-(0, 0) source pixel, and which kernel rows / columns of the
  // taps fall inside the image (bit k: row / column k; no bits for a lane
  // without a pixel, or a block past the range)
  struct Blk {
    uint32_t pix_out, b0, b1, cg;
    uint32_t rows, cols;
    bool valid;
  };
  auto decode = [&](uint32_t item, bool in_range) {
    Blk b;
    const uint32_t blk = item / a.ncg;
    b.cg = item - blk * a.ncg;
    b.pix_out = blk * 32 + l32;
    b.valid = b.pix_out < a.M;
    const uint32_t pp = b.valid ? b.pix_out : 0;
    const uint32_t img = fdiv(pp, a.fd_ohw);
    const uint32_t rem = pp - img * a.OHW;
    const uint32_t oy = fdiv(rem, a.fd_ow);
    const uint32_t ox = rem - oy * a.OW;
    const int32_t iy0 = (int32_t)(oy * a.S) - a.PT;
    const int32_t ix0 = (int32_t)(ox * a.S) - a.PL;
    constexpr int KS = TAPS == 9 ? 3 : 1;
    uint32_t rows = 0, cols = 0;
#pragma unroll
    for (int k = 0; k < KS; ++k) {
      rows |= (uint32_t)((uint32_t)(iy0 + k * (int32_t)a.D) < a.IH) << k;
      cols |= (uint32_t)((uint32_t)(ix0 + k * (int32_t)a.D) < a.IW) << k;
    }
    b.rows = (b.valid & in_range) ? rows : 0u;
    b.cols = cols;
    // wraps (unsigned) when the tap-(0, 0) pixel lies above or left of the
    // image; tap offsets bring in-image taps back, the others are not read
    const uint32_t pix = (img * a.IH + (uint32_t)iy0) * a.IW + (uint32_t)ix0;
    b.b0 = pix * a.stride_u[0] + a.off_u[0];
    b.b1 = pix * a.stride_u[1] + a.off_u[1];
    return b;
  };
  // a lane's source of one tap: both parts' unit index of its pixel, or
  // ok = false (outside the image, or no pixel) for zeros
  struct TapSrc {
    uint32_t b0, b1;
    bool ok;
  };
  auto tap_src = [&](const Blk &b, int tap) {
    TapSrc t;
    const int ky = tap / 3, kx = tap % 3;
    t.ok = ((b.rows >> ky) & (b.cols >> kx) & 1u) != 0;
    const uint32_t dpix = (uint32_t)ky * a.D * a.IW + (uint32_t)kx * a.D;
    t.b0 = b.b0 + dpix * a.stride_u[0];
    t.b1 = b.b1 + dpix * a.stride_u[1];
    return t;
  };
  // the MFMA operand of step j: unit 2(j - part start) + lh of step j's part
  auto load_step = [&](const TapSrc &t, int j) {
    const bool p1 = (uint32_t)j >= nj0;
    const uint32_t u = 2 * ((uint32_t)j - (p1 ? nj0 : 0u)) + lh;
    const bool in = t.ok & (u < (p1 ? a.nu[1] : a.nu[0]));
    const uint32_t off = in ? ((p1 ? t.b1 : t.b0) + u) * 16u : kOob;
    return __builtin_amdgcn_raw_buffer_load_b128(p1 ? rs1 : rs0, off, 0, 0);
  };
  // the lane's weight operands of step s (tap s / NJ, step s % NJ); wlo is
  // wl passed through an empty asm once per block, so the compiler cannot
  // hoist the (loop-invariant) reads out of the block loop into registers
  uint32_t wlo = wl;
  auto load_w = [&](int s, u32x4 (&w)[NOB]) {
#pragma unroll
    for (int o = 0; o < NOB; ++o) w[o] = Wl[wlo + s * 2 * RS + o * 32];
  };

  // Software pipeline over the TAPS * NJ MFMA steps of each block: a ring of D
  // operand registers (D divides TAPS * NJ, so step s of every block uses slot
  // s % D); right after step s's MFMAs its slot is refilled with step s + D
  // -- of the next block for the last D steps -- so D - 1 steps of MFMAs
  // cover every load, across block ends too. Within a block the weights of
  // step s + 1 are read from LDS before step s's MFMAs.
  constexpr int NS = TAPS * NJ;
  static_assert(NS % D == 0, "operand ring");
  uint32_t blk = b_begin + wave;
  if (blk >= b_end) return;
  Blk cur = decode(blk, true);
  u32x4 x[D];
  TapSrc ts = tap_src(cur, 0);
#pragma unroll
  for (int s = 0; s < D; ++s) {
    if (s > 0 && s % NJ == 0) ts = tap_src(cur, s / NJ);
    x[s] = load_step(ts, s % NJ);
  }
  for (;;) {
    wlo = wl + cur.cg * NC;
    __asm__ volatile("" : "+v"(wlo));
    u32x4 wv[2][NOB];
    load_w(0, wv[0]);
    const uint32_t blk_next = blk + kWaves;
    const bool more = blk_next < b_end;
    // past the range the next block reads zeros (offsets outside the
    // buffers): the ring's loads are issued unconditionally, so the block
    // loop has no divergent branch and never drains the ring
    const Blk nxt = decode(more ? blk_next : blk, more);
    f32x16 acc[NOB];
#pragma unroll
    for (int o = 0; o < NOB; ++o) acc[o] = f32x16{};
    // a block's MFMA steps at raised priority, its epilogue (LDS staging,
    // stores) at the normal one: the SIMD's wavefronts in their MFMA loops
    // issue ahead of one in its epilogue (C3a 45 -> 43 us, C3b 129 -> 125 us,
    // one box, graph-replayed)
    __builtin_amdgcn_s_setprio(1);
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      if (s + 1 < NS) load_w(s + 1, wv[(s + 1) & 1]);
      const u32x4 xs = x[s % D];
#pragma unroll
      for (int o = 0; o < NOB; ++o) {
        const u32x4 w = wv[s & 1][o];
        if constexpr (F32) {
          const f32x4 w4 = __builtin_bit_cast(f32x4, w), x4 = __builtin_bit_cast(f32x4, xs);
#pragma unroll
          for (int c = 0; c < 4; ++c) acc[o] = __builtin_amdgcn_mfma_f32_32x32x2f32(w4[c], x4[c], acc[o], 0, 0, 0);
        } else if constexpr (DT == DT_F16) {
          acc[o] = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, w), __builtin_bit_cast(f16x8, xs),
                                                         acc[o], 0, 0, 0);
        } else {
          acc[o] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, w),
                                                          __builtin_bit_cast(bf16x8, xs), acc[o], 0, 0, 0);
        }
      }
      // refill: step s + D, a new tap's source when it starts one
      const int sl = s + D;
      if (sl < NS) {
        if (sl % NJ == 0) ts = tap_src(cur, sl / NJ);
        x[s % D] = load_step(ts, sl % NJ);
      } else {
        if ((sl - NS) % NJ == 0) ts = tap_src(nxt, (sl - NS) / NJ);
        x[s % D] = load_step(ts, (sl - NS) % NJ);
      }
      // keep the scheduler from hoisting later steps' reads (registers)
      __builtin_amdgcn_sched_barrier(0);
    }
    __builtin_amdgcn_s_setprio(0);

    if (a.st_off) {
      // through the wavefront's LDS rows: act(acc + bias) in the MFMA
      // layout, then 8 pixels x 8 four-channel pieces per store, so a store
      // instruction writes whole contiguous rows (one 4 KB run for 32 fp32
      // channels) instead of 16 bytes at each of 64 pixels
      float *rows = reinterpret_cast<float *>(lds + a.st_off) + wave * 32 * kStPitch;
      const uint32_t pix0 = cur.pix_out - l32;
#pragma unroll
      for (int o = 0; o < NOB; ++o) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const uint32_t cl = 8 * q + 4 * lh;
          const uint32_t c = cur.cg * NC + o * 32 + cl;
          f32x4 v = f32x4{acc[o][4 * q], acc[o][4 * q + 1], acc[o][4 * q + 2], acc[o][4 * q + 3]} +
                    *reinterpret_cast<const f32x4 *>(Bl + c);
          *reinterpret_cast<f32x4 *>(rows + l32 * kStPitch + cl) = act4(actp, v);
        }
        __builtin_amdgcn_wave_barrier();
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const uint32_t px = 8 * i + (lane >> 3), pc = 4 * (lane & 7);
          const uint32_t m = pix0 + px, c = cur.cg * NC + o * 32 + pc;
          f32x4 v = *reinterpret_cast<const f32x4 *>(rows + px * kStPitch + pc);
          if (m < a.M && c < a.N4) {
            const size_t vi = (size_t)m * (a.N4 / 4) + c / 4;
            if (a.has_res) v += Vec4IO<DT>::load(a.res, vi);
            Vec4IO<DT>::store(a.y, vi, v);
          }
        }
        __builtin_amdgcn_wave_barrier();
      }
    } else if (cur.valid) {
#pragma unroll
      for (int o = 0; o < NOB; ++o) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const uint32_t c = cur.cg * NC + o * 32 + 8 * q + 4 * lh;
          if (c >= a.N4) continue;
          f32x4 v = f32x4{acc[o][4 * q], acc[o][4 * q + 1], acc[o][4 * q + 2], acc[o][4 * q + 3]} +
                    *reinterpret_cast<const f32x4 *>(Bl + c);
          v = act4(actp, v);
          const size_t vi = (size_t)cur.pix_out * (a.N4 / 4) + c / 4;
          if (a.has_res) v += Vec4IO<DT>::load(a.res, vi);
          Vec4IO<DT>::store(a.y, vi, v);
        }
      }
    }
    if (!more) break;
    blk = blk_next;
    cur = nxt;
  }
}

template <int DT, int NOB, int TAPS, int NJ, int D>
hipError_t launch_inst(const IgDirectArgs &a, hipStream_t st) {
  static const hipError_t attr =
      hipFuncSetAttribute(reinterpret_cast<const void *>(conv_igemm_direct_kernel<DT, NOB, TAPS, NJ, D>),
                          hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
  if (attr != hipSuccess) return attr;
  // the output staging rows go after the weights and biases where LDS has room
  IgDirectArgs b = a;
  const uint32_t base = ig_direct_lds_bytes(TAPS, a.nj, a.N4);
  b.st_off = base + kStBytes <= 160u * 1024u ? base : 0u;
  const uint32_t lds = base + (b.st_off ? kStBytes : 0u);
  const uint32_t grid = ig_direct_grid(a.nblk, a.nj, a.N4);
  hipLaunchKernelGGL((conv_igemm_direct_kernel<DT, NOB, TAPS, NJ, D>), dim3(grid), dim3(kIgDirectThreads), lds, st, b);
  return hipGetLastError();
}

template <int DT, int NOB, bool PW_ONLY = false>
hipError_t launch_nob(const IgDirectArgs &a, hipStream_t st) {
  // operand ring depth D (a divisor of 9 * NJ): 6 / 9 / 12 steps, measured
  // against 3 and 18 on the 16 -> 32 and 32 -> 32 / 64 shapes
  if (PW_ONLY || a.taps == 1) {
    // 1x1: the steps run up to the instantiation's count (ring 8 / 12 deep)
    switch (pw_lds_steps(a.nj)) {
      case 8: return launch_inst<DT, NOB, 1, 8, 8>(a, st);
      case 12: return launch_inst<DT, NOB, 1, 12, 12>(a, st);
      case 16: return launch_inst<DT, NOB, 1, 16, 8>(a, st);
      case 24: return launch_inst<DT, NOB, 1, 24, 12>(a, st);
      case 32: return launch_inst<DT, NOB, 1, 32, 8>(a, st);
      default: return hipErrorInvalidValue;
    }
  }
  if constexpr (PW_ONLY) return hipErrorInvalidValue;
  switch (a.nj) {
    case 1: return launch_inst<DT, NOB, 9, 1, 9>(a, st);
    case 2: return launch_inst<DT, NOB, 9, 2, 6>(a, st);
    case 3: return launch_inst<DT, NOB, 9, 3, 9>(a, st);
    case 4: return launch_inst<DT, NOB, 9, 4, 12>(a, st);
    case 5: return launch_inst<DT, NOB, 9, 5, 9>(a, st);
    case 6: return launch_inst<DT, NOB, 9, 6, 9>(a, st);
    case 7: return launch_inst<DT, NOB, 9, 7, 9>(a, st);
    case 8: return launch_inst<DT, NOB, 9, 8, 9>(a, st);
    case 9: return launch_inst<DT, NOB, 9, 9, 9>(a, st);
    case 10: return launch_inst<DT, NOB, 9, 10, 9>(a, st);
    default: return hipErrorInvalidValue;
  }
}

template <int DT>
hipError_t launch_dt(const IgDirectArgs &a, hipStream_t st) {
  switch (ig_direct_nob(a.N4)) {
    case 1: return launch_nob<DT, 1>(a, st);
    case 2: return launch_nob<DT, 2>(a, st);
    default:
      // four blocks: fp32 pointwise only (wider 16-bit and 3x3 calls are
      // planned elsewhere)
      if constexpr (DT == DT_F32) return launch_nob<DT, 4, true>(a, st);
      return hipErrorInvalidValue;
  }
}

}  // namespace

hipError_t launch_ig_direct(const IgDirectArgs &a, int dt, hipStream_t st) {
  if (a.N4 == 0 || a.N4 % 4 || a.N4 > (a.taps == 1 ? 256u : 64u) || a.ncg != ig_direct_ncg(a.N4) || a.nj == 0 ||
      a.nj0 > a.nj || (a.taps != 1 && a.taps != 9) ||
      (a.taps == 9 && a.nj > kIgDirectMaxSteps) || (a.taps == 1 && pw_lds_steps(a.nj) == 0) ||
      ig_direct_lds_bytes(a.taps, a.nj, a.N4) > 160u * 1024u)
    return hipErrorInvalidValue;
  switch (dt) {
    case DT_F32: return launch_dt<DT_F32>(a, st);
    case DT_F16: return launch_dt<DT_F16>(a, st);
    case DT_BF16: return launch_dt<DT_BF16>(a, st);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace aih
