// dw_pw_impl.h -- the fused depthwise KxK conv + pointwise 1x1 conv kernel
// (dw_pw.hip: its design, planner and C ABI), templated on the storage dtype
// so that the fp32 and 16-bit instantiations build in separate translation
// units.
#pragma once

#include <hip/hip_runtime.h>

#include "dw_pw.h"

namespace aih {

typedef __attribute__((address_space(3))) void dp_lds_void;
constexpr uint32_t kOob = 0x80000000u;  // a byte offset past every buffer the kernel reads (< 2 GiB)

__device__ __forceinline__ __amdgpu_buffer_rsrc_t dp_rsrc(const void *base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), 0, (int)bytes, 0x00020000);
}

// One 16-byte LDS-direct load per lane: lane i's bytes land at dst + 16 i.
__device__ __forceinline__ void dp_load16(__amdgpu_buffer_rsrc_t rs, char *dst, uint32_t off, uint32_t soff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (dp_lds_void *)dst, 16, off, (int)soff, 0, 0);
}

// DT: storage dtype; K: depthwise kernel size; S: stride; NO: blocks of 16
// output channels; U: 16-byte units (4 fp32 / 8 16-bit channels) per chunk
// and halo pixel; NB: output rows (16-pixel row blocks) per wavefront, 4 or
// 2; CL: both activations are clamp-type (one v_med3 each, no mode switch).
template <int DT, int K, int S, int NO, int U, int NB, bool CL>
__global__ __launch_bounds__(512) void dw_pw_kernel(DwPwArgs a) {
  constexpr bool F32 = DT == DT_F32;
  constexpr uint32_t ES = F32 ? 4 : 2, CPU = 16 / ES, EC = CPU * U, COP = 16 * NO, PITCH = (U + 1) * 16;
  constexpr int HR = (NB - 1) * S + K;  // halo rows one wavefront reads
  constexpr int XS = dwpw_slots(S);
  constexpr uint32_t NWD = K * K * U, NWP = U * COP;  // weight slots of a chunk
  extern __shared__ __align__(16) char lds[];
  const uint32_t tid = threadIdx.x, lane = tid & 63, p16 = lane & 15, kq = lane >> 4;
  const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const uint32_t nthr = blockDim.x, nwaves = nthr >> 6;
  const uint32_t wxi = wave % a.wx, wyi = wave / a.wx;

  // ---- this workgroup's tile ----
  const uint32_t T = xcd_remap(blockIdx.x, gridDim.x, a.nxcd);
  const uint32_t img = fdiv(T, a.fd_pi);
  const uint32_t trem = T - img * a.per_img;
  const uint32_t tyi = fdiv(trem, a.fd_tx);
  const uint32_t ty0 = tyi * a.TH, tx0 = (trem - tyi * a.tiles_x) * a.TW;
  const int32_t iy0 = (int32_t)(ty0 * S) - a.PT, ix0 = (int32_t)(tx0 * S) - a.PL;

  // ---- this thread's halo slots (the same for every chunk) ----
  // slot s = 64 (wave + nwaves k) + lane holds unit s % (U + 1) of halo
  // pixel s / (U + 1) (unit U: the pad; slots past the halo pad the region
  // to whole rows of 64); gsl[k]: the unit's byte offset in the image for
  // channel 0 of a chunk (the chunk's channel offset goes in the scalar
  // offset), or kOob (outside the image, the pad, past the halo). (At 16
  // bit a pixel's bytes need not be a multiple of 16, so the offset cannot
  // carry the unit index in its low bits; the last chunk recomputes it.)
  const uint32_t nrows = (a.xrows + nwaves - 1 - wave) / nwaves;  // uniform: 64-slot rows this wavefront copies
  uint32_t gsl[XS];
#pragma unroll
  for (int k = 0; k < XS; ++k) {
    const uint32_t s = 64 * (wave + nwaves * k) + lane;
    const uint32_t P = s / (U + 1), u = s - P * (U + 1);
    const uint32_t hr = fdiv(P, a.fd_hw), hc = P - hr * a.HW;
    uint32_t hx = hc;
    if constexpr (S == 2) hx = hc < a.HWE ? 2 * hc : 2 * (hc - a.HWE) + 1;
    const uint32_t iy = (uint32_t)(iy0 + (int32_t)hr), ix = (uint32_t)(ix0 + (int32_t)hx);
    gsl[k] = (u < U && hr < a.HH && iy < a.IH && ix < a.IW) ? (iy * a.IW + ix) * a.C * ES + 16 * u : kOob;
  }

  // the weight copies go out in 64-slot rows, row r from wavefront
  // (first + r) % nwaves: this wavefront's first row
  auto first_row = [&](uint32_t first) { return (wave + nwaves - first % nwaves) % nwaves; };

  // chunk c (channels [EC c, EC c + EC)) -> LDS buffer b
  auto stage = [&](uint32_t c, uint32_t b) {
    char *B = lds + b * a.buf_bytes;
    const uint32_t c0 = c * EC, soff = c0 * ES;
    const __amdgpu_buffer_rsrc_t rs_x = dp_rsrc((const char *)a.x + (size_t)img * a.img_bytes, a.img_bytes);
    if (c0 + EC <= a.C) {
#pragma unroll
      for (int k = 0; k < XS; ++k) {
        if ((uint32_t)k >= nrows) break;
        dp_load16(rs_x, B + 1024 * (wave + nwaves * k), gsl[k], soff);
      }
    } else {
      // the last chunk of a C that is no multiple of EC: units past C read
      // zeros (a unit reaching past C -- 16-bit, C % 8 = 4 -- reads the next
      // pixel's first channels, finite values whose projection weights are
      // zero)
#pragma unroll
      for (int k = 0; k < XS; ++k) {
        if ((uint32_t)k >= nrows) break;
        const uint32_t u = (64 * (wave + nwaves * k) + lane) % (U + 1);
        dp_load16(rs_x, B + 1024 * (wave + nwaves * k), c0 + CPU * u < a.C ? gsl[k] : kOob, soff);
      }
    }
    // depthwise weights [tap][U units], its bias [U units], pointwise weights [U groups][COP rows]
    char *W = B + a.off_wd;
    const __amdgpu_buffer_rsrc_t rs_wd = dp_rsrc(a.wd, K * K * a.C * ES);
    for (uint32_t s0 = 64 * first_row(1); s0 < NWD; s0 += nthr) {
      const uint32_t s = s0 + lane;
      if (s < NWD) {
        const uint32_t t = s / U, u = s % U;
        dp_load16(rs_wd, W + s0 * 16, c0 + CPU * u < a.C ? (t * a.C + CPU * u) * ES : kOob, soff);
      }
    }
    if (wave == 0 && lane < U) {
      const __amdgpu_buffer_rsrc_t rs_bd = dp_rsrc(a.bd, a.C * ES);
      dp_load16(rs_bd, W + NWD * 16, c0 + CPU * lane < a.C ? 16 * lane : kOob, soff);
    }
    // fp32: item s = (group g of 4 K, output channel o), one 16-byte group;
    // 16-bit: item s = (group g, channel pair 2 o2 .. 2 o2 + 1), two 8-byte
    // groups -- row g of COP channels either way ([K group][COP][4], packed)
    const __amdgpu_buffer_rsrc_t rs_wp = dp_rsrc(a.wp, a.KGP * a.CO4 * 4 * ES);
    constexpr uint32_t RI = F32 ? COP : COP / 2;  // 16-byte items per K-group row
    for (uint32_t s0 = 64 * first_row(2); s0 < NWP; s0 += nthr) {
      const uint32_t s = s0 + lane;
      if (s < NWP) {
        const uint32_t g = s / RI, o = s % RI;
        const bool ok = o * (F32 ? 1 : 2) < a.CO4 && c0 + 4 * g < a.C;
        dp_load16(rs_wp, W + (NWD + U + s0) * 16, ok ? (g * a.CO4 * 4 * ES + o * 16) : kOob, c0 * a.CO4 * ES);
      }
    }
  };

  // LDS byte offset of this lane's halo pixel for tap (0, 0) of its first
  // block, unit kq (stride 2: halo columns stored even first)
  const uint32_t xbase = ((wyi * NB * S) * a.HW + 16 * wxi + p16) * PITCH + kq * 16;

  f32x4 acc[NB][NO];
#pragma unroll
  for (int b = 0; b < NB; ++b)
#pragma unroll
    for (int o = 0; o < NO; ++o) acc[b][o] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  const Act actd = act_params(a.act_d), actp = act_params(a.act_p);

  // chunk c lives in buffer c % 2; chunk c + 1 goes out once every
  // wavefront is done with chunk c - 1 (the barrier), into that buffer
  const uint32_t nch = a.nchunks;
  stage(0, 0);
  for (uint32_t c = 0; c < nch; ++c) {
    // this wavefront's copies of chunk c have landed, then the barrier
    // publishes every wavefront's
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0); expcnt, lgkmcnt untouched
    __syncthreads();
    if (c + 1 < nch) stage(c + 1, (c + 1) & 1);
    const uint32_t cur = c & 1;
    const char *B = lds + cur * a.buf_bytes;
    const char *W = B + a.off_wd;
    // lane group kq takes unit kq of the chunk (and kq + 4, ... for U > 4)
#pragma unroll
    for (int h = 0; h < U / 4; ++h) {
      const uint32_t u = 4 * h + kq;
      if constexpr (F32) {
        f32x4 w[K * K];
#pragma unroll
        for (int t = 0; t < K * K; ++t) w[t] = *reinterpret_cast<const f32x4 *>(W + (t * U + u) * 16);
        const f32x4 bias = *reinterpret_cast<const f32x4 *>(W + (NWD + u) * 16);
        f32x4 d[NB];
#pragma unroll
        for (int b = 0; b < NB; ++b) d[b] = bias;
        // halo row i feeds block b with kernel row i - S b
#pragma unroll
        for (int i = 0; i < HR; ++i) {
#pragma unroll
          for (int kx = 0; kx < K; ++kx) {
            const uint32_t col = S == 1 ? (uint32_t)kx : (uint32_t)(kx & 1) * a.HWE + (uint32_t)(kx >> 1);
            const f32x4 xv = *reinterpret_cast<const f32x4 *>(B + xbase + h * 64 + (i * a.HW + col) * PITCH);
#pragma unroll
            for (int b = 0; b < NB; ++b) {
              const int ky = i - S * b;
              if (ky >= 0 && ky < K) d[b] += xv * w[ky * K + kx];
            }
          }
        }
#pragma unroll
        for (int b = 0; b < NB; ++b) {
          if constexpr (CL) {
#pragma unroll
            for (int j = 0; j < 4; ++j) d[b][j] = act_clamp_any(actd, d[b][j]);
          } else {
            d[b] = act4(actd, d[b]);
          }
        }
        f32x4 aw[NO];
#pragma unroll
        for (int o = 0; o < NO; ++o)
          aw[o] = *reinterpret_cast<const f32x4 *>(W + (NWD + U + u * COP + 16 * o + p16) * 16);
        // the projection MFMAs at raised priority: a wavefront that has
        // finished its depthwise issues them ahead of the SIMD's others still
        // in theirs (C4 chain, fp32: 800 -> 770 us on one box; the 16-bit
        // branch below measured no gain from it)
        __builtin_amdgcn_s_setprio(1);
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
          for (int b = 0; b < NB; ++b)
#pragma unroll
            for (int o = 0; o < NO; ++o)
              acc[b][o] = __builtin_amdgcn_mfma_f32_16x16x4f32(aw[o][j], d[b][j], acc[b][o], 0, 0, 0);
        __builtin_amdgcn_s_setprio(0);
      } else {
        // 16-bit storage: the depthwise in fp32 from the widened taps (sum
        // from the bias, taps in (ky, kx) order), act, rounded to DT where
        // the unfused depthwise stores its output; that is the B operand of
        // v_mfma_f32_16x16x32 (K slice kq = the unit's 8 channels), the
        // projection weights of those channels the A operand (K groups 2u
        // and 2u + 1, rows of COP channels)
        float w[K * K][8];
#pragma unroll
        for (int t = 0; t < K * K; ++t) {
          const u32x4 wr = *reinterpret_cast<const u32x4 *>(W + (t * U + u) * 16);
          const f32x4 lo = unpack4<DT>(u32x2{wr.x, wr.y}), hi = unpack4<DT>(u32x2{wr.z, wr.w});
#pragma unroll
          for (int j = 0; j < 4; ++j) w[t][j] = lo[j], w[t][4 + j] = hi[j];
        }
        const u32x4 br = *reinterpret_cast<const u32x4 *>(W + (NWD + u) * 16);
        const f32x4 blo = unpack4<DT>(u32x2{br.x, br.y}), bhi = unpack4<DT>(u32x2{br.z, br.w});
        float d[NB][8];
#pragma unroll
        for (int b = 0; b < NB; ++b)
#pragma unroll
          for (int j = 0; j < 4; ++j) d[b][j] = blo[j], d[b][4 + j] = bhi[j];
#pragma unroll
        for (int i = 0; i < HR; ++i) {
#pragma unroll
          for (int kx = 0; kx < K; ++kx) {
            const uint32_t col = S == 1 ? (uint32_t)kx : (uint32_t)(kx & 1) * a.HWE + (uint32_t)(kx >> 1);
            const u32x4 xr = *reinterpret_cast<const u32x4 *>(B + xbase + h * 64 + (i * a.HW + col) * PITCH);
            const f32x4 xlo = unpack4<DT>(u32x2{xr.x, xr.y}), xhi = unpack4<DT>(u32x2{xr.z, xr.w});
            float xv[8];
#pragma unroll
            for (int j = 0; j < 4; ++j) xv[j] = xlo[j], xv[4 + j] = xhi[j];
#pragma unroll
            for (int b = 0; b < NB; ++b) {
              const int ky = i - S * b;
              if (ky >= 0 && ky < K) {
#pragma unroll
                for (int j = 0; j < 8; ++j) d[b][j] = __builtin_fmaf(xv[j], w[ky * K + kx][j], d[b][j]);
              }
            }
          }
        }
        u32x4 bop[NB];
#pragma unroll
        for (int b = 0; b < NB; ++b) {
          if constexpr (CL) {
#pragma unroll
            for (int j = 0; j < 8; ++j) d[b][j] = act_clamp_any(actd, d[b][j]);
          } else {
            act_array<8>(actd, d[b]);
          }
          const u32x2 lo = pack4<DT>(f32x4{d[b][0], d[b][1], d[b][2], d[b][3]});
          const u32x2 hi = pack4<DT>(f32x4{d[b][4], d[b][5], d[b][6], d[b][7]});
          bop[b] = u32x4{lo.x, lo.y, hi.x, hi.y};
        }
        const char *wrow = W + (NWD + U) * 16 + (2 * u * COP + p16) * 8;
#pragma unroll
        for (int o = 0; o < NO; ++o) {
          const u32x2 lo = *reinterpret_cast<const u32x2 *>(wrow + 16 * o * 8);
          const u32x2 hi = *reinterpret_cast<const u32x2 *>(wrow + 16 * o * 8 + COP * 8);
          const u32x4 aw = u32x4{lo.x, lo.y, hi.x, hi.y};
#pragma unroll
          for (int b = 0; b < NB; ++b) {
            if constexpr (DT == DT_F16)
              acc[b][o] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, aw),
                                                                 __builtin_bit_cast(f16x8, bop[b]), acc[b][o], 0, 0, 0);
            else
              acc[b][o] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, aw),
                                                                  __builtin_bit_cast(bf16x8, bop[b]), acc[b][o], 0, 0,
                                                                  0);
          }
        }
      }
    }
  }

  // ---- epilogue: lane holds output channels 16 o + 4 kq .. + 3 of pixel p16 of each block ----
  f32x4 bp[NO];
#pragma unroll
  for (int o = 0; o < NO; ++o) {
    const uint32_t ch = 16 * o + 4 * kq;
    bp[o] = ch < a.CO4 ? Vec4IO<DT>::load(a.bp, ch / 4) : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  }
  const uint32_t ox = tx0 + 16 * wxi + p16;
#pragma unroll
  for (int b = 0; b < NB; ++b) {
    const uint32_t oy = ty0 + wyi * NB + b;
    if (oy >= a.OH || ox >= a.OW) continue;
    const size_t pix = ((size_t)img * a.OH + oy) * a.OW + ox;
#pragma unroll
    for (int o = 0; o < NO; ++o) {
      const uint32_t ch = 16 * o + 4 * kq;
      if (ch >= a.CO4) continue;
      f32x4 v = acc[b][o] + bp[o];
      if constexpr (CL) {
#pragma unroll
        for (int j = 0; j < 4; ++j) v[j] = act_clamp_any(actp, v[j]);
      } else {
        v = act4(actp, v);
      }
      const size_t vi = pix * (a.CO4 / 4) + ch / 4;
      if (a.has_res) v += Vec4IO<DT>::load(a.res, vi);
      Vec4IO<DT>::store(a.y, vi, v);
    }
  }
}

template <int DT, int K, int S, int NO, int NB, bool CL>
hipError_t dp_prepare_inst() {
  static const hipError_t e =
      hipFuncSetAttribute(reinterpret_cast<const void *>(dw_pw_kernel<DT, K, S, NO, kDpUnits, NB, CL>),
                          hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
  return e;
}

template <int DT, int K, int S, int NO, int NB, bool CL>
hipError_t dp_launch_inst(const DwPwArgs &a, uint32_t waves, uint32_t lds, uint32_t grid, hipStream_t st) {
  const hipError_t e = dp_prepare_inst<DT, K, S, NO, NB, CL>();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL((dw_pw_kernel<DT, K, S, NO, kDpUnits, NB, CL>), dim3(grid), dim3(64 * waves), lds, st, a);
  return hipGetLastError();
}

// Workgroups per CU, or -1 when the runtime cannot answer (no device).
template <int DT, int K, int S, int NO, int NB, bool CL>
int dp_occ_inst(uint32_t waves, uint32_t lds) {
  if (dp_prepare_inst<DT, K, S, NO, NB, CL>() != hipSuccess) return -1;
  int per_cu = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, dw_pw_kernel<DT, K, S, NO, kDpUnits, NB, CL>,
                                                   (int)(64 * waves), lds) != hipSuccess)
    return -1;
  return per_cu;
}

#define AIH_DP_SHAPES(X) \
  X(3, 1, 1) X(3, 1, 2) X(3, 1, 3) X(3, 1, 4) X(3, 2, 1) X(3, 2, 2) X(3, 2, 3) X(3, 2, 4)

// The instantiations of one dtype, by shape: rows 2 or 4, cl both
// activations clamp-type.
template <int DT>
hipError_t dp_launch_dt(const DwPwArgs &a, uint32_t k, uint32_t s, uint32_t rows, uint32_t waves, uint32_t lds,
                        uint32_t grid, hipStream_t st) {
  const uint32_t no = dwpw_no(a.CO4);
  const bool cl = act_is_clamp(a.act_d) && act_is_clamp(a.act_p);
#define AIH_DP_LAUNCH(K_, S_, NO_)                                                                  \
  if (k == K_ && s == S_ && no == NO_) {                                                            \
    if (rows == 2)                                                                                  \
      return cl ? dp_launch_inst<DT, K_, S_, NO_, 2, true>(a, waves, lds, grid, st)                 \
                : dp_launch_inst<DT, K_, S_, NO_, 2, false>(a, waves, lds, grid, st);               \
    if (rows == 4)                                                                                  \
      return cl ? dp_launch_inst<DT, K_, S_, NO_, 4, true>(a, waves, lds, grid, st)                 \
                : dp_launch_inst<DT, K_, S_, NO_, 4, false>(a, waves, lds, grid, st);               \
  }
  AIH_DP_SHAPES(AIH_DP_LAUNCH)
#undef AIH_DP_LAUNCH
  return hipErrorInvalidValue;
}

// -2: no instantiation; -1: no device to ask; else workgroups per CU.
template <int DT>
int dp_occ_dt(uint32_t k, uint32_t s, uint32_t no, uint32_t rows, bool cl, uint32_t waves, uint32_t lds) {
#define AIH_DP_OCC(K_, S_, NO_)                                                                                 \
  if (k == K_ && s == S_ && no == NO_)                                                                          \
    return rows == 2 ? (cl ? dp_occ_inst<DT, K_, S_, NO_, 2, true>(waves, lds)                                  \
                           : dp_occ_inst<DT, K_, S_, NO_, 2, false>(waves, lds))                                \
                     : (cl ? dp_occ_inst<DT, K_, S_, NO_, 4, true>(waves, lds)                                  \
                           : dp_occ_inst<DT, K_, S_, NO_, 4, false>(waves, lds));
  AIH_DP_SHAPES(AIH_DP_OCC)
#undef AIH_DP_OCC
  return -2;
}

}  // namespace aih
