// ir_block_impl.h -- fused inverted-residual block for gfx950 (CDNA4).
//
// Three consecutive SwOp::Conv that the reference lowers to three separate
// dispatches (crates/ai-gpu-runtime/src/lowering.rs:122-152: GemmPwSpec,
// ConvDwSpec, GemmPwSpec) run as one kernel, so the 4x-expanded intermediate
// never leaves the CU:
//
//   e = act_e(x . We + be)            1x1 expand, C -> E      (MFMA)
//   d = act_d(dw3x3_S(e) + bd)        depthwise, stride S     (VALU, fp32)
//   y = act_p(d . Wp + bp) (+ res)    1x1 project, E -> CO    (MFMA)
//
// with each stage's arithmetic and rounding matching its unfused kernel:
// fp32 accumulation, bias -> act -> (+ residual) as in common/epilogue.rs:13-30,
// and the e and d intermediates rounded to the storage dtype exactly where the
// unfused path stores them.
//
// Work decomposition. A workgroup (4 wavefronts) owns a TH x TW tile of output
// pixels of one image and walks E in chunks of EC channels:
//   (0) the input tile with its halo, HH x HW pixels x C channels, is copied
//       to LDS once per tile (zeros outside the image);
//   (1) expand: [halo px x C] x [C x EC] on MFMA, in 32-pixel x 32-channel
//       blocks dealt round-robin to the wavefronts; bias + act in the MFMA
//       layout; halo pixels outside the image are set to 0 (they are the
//       depthwise zero padding, not expand(0)); the chunk is stored to LDS;
//   (2) depthwise + project: every wavefront owns NPW 32-pixel blocks of the
//       output tile. Lane l computes the depthwise output of pixel l%32 for
//       the K slice that lane l feeds to the projection MFMA, so the
//       depthwise result is the MFMA B operand directly, without a round
//       trip through LDS. The projection accumulates over all chunks in
//       registers: NPW x NOB 32x32 fp32 blocks per wavefront.
// After the last chunk: bias, act, residual and the store to HBM.
//
// MFMA operand convention (as in the conv-GEMM kernel): the weights are the A
// operand (rows = output channels), the pixels the B operand; every operand
// is one 16-byte LDS read per lane at row (l%32), K offset ks*KSTEP + (l/32)*KSTEP/2:
//   f16/bf16: v_mfma_f32_32x32x16_{f16,bf16}, KSTEP = 16, one MFMA per read;
//   fp32:     v_mfma_f32_32x32x2f32,          KSTEP = 8,  four MFMAs per read
//             (MFMA c takes component c: K = 4*(l/32) + c for both operands).
// Result lane l holds pixel l%32 and channels 8*(r/4) + 4*(l/32) + r%4.
// LDS rows are padded by 16 bytes so that 8 consecutive lanes reading 16 bytes
// of 8 consecutive rows hit 32 distinct banks.
#pragma once

#include "aih_device.h"
#include "ir_block.h"

namespace aih {

// Expanded channels per chunk.
constexpr int IR_EC = 32;

template <int DT>
__device__ __forceinline__ f32x16 ir_mma(u32x4 a, u32x4 b, f32x16 c) {
  if constexpr (DT == DT_F16) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c,
                                                  0, 0, 0);
  } else if constexpr (DT == DT_BF16) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b),
                                                   c, 0, 0, 0);
  } else {
    const f32x4 fa = __builtin_bit_cast(f32x4, a), fb = __builtin_bit_cast(f32x4, b);
#pragma unroll
    for (int k = 0; k < 4; ++k) c = __builtin_amdgcn_mfma_f32_32x32x2f32(fa[k], fb[k], c, 0, 0, 0);
    return c;
  }
}

// 16 bytes of storage <-> HK fp32 values (HK = 8 for 16-bit, 4 for fp32).
template <int DT, int HK>
__device__ __forceinline__ void ir_unpack(u32x4 v, float (&out)[HK]) {
  if constexpr (DT == DT_F32) {
    const f32x4 f = __builtin_bit_cast(f32x4, v);
    out[0] = f.x; out[1] = f.y; out[2] = f.z; out[3] = f.w;
  } else {
    const f32x4 lo = unpack4<DT>(u32x2{v.x, v.y}), hi = unpack4<DT>(u32x2{v.z, v.w});
    out[0] = lo.x; out[1] = lo.y; out[2] = lo.z; out[3] = lo.w;
    out[4] = hi.x; out[5] = hi.y; out[6] = hi.z; out[7] = hi.w;
  }
}

template <int DT, int HK>
__device__ __forceinline__ u32x4 ir_pack(const float (&v)[HK]) {
  if constexpr (DT == DT_F32) {
    return __builtin_bit_cast(u32x4, f32x4{v[0], v[1], v[2], v[3]});
  } else {
    const u32x2 lo = pack4<DT>(f32x4{v[0], v[1], v[2], v[3]});
    const u32x2 hi = pack4<DT>(f32x4{v[4], v[5], v[6], v[7]});
    return u32x4{lo.x, lo.y, hi.x, hi.y};
  }
}

// d[j] += x[j] * w[j] for the HK channels in 16 bytes of x and of w (both in
// the storage dtype; f16 products go through v_fma_mix_f32, fp32 accumulate).
template <int DT, int HK>
__device__ __forceinline__ void ir_fma_taps(u32x4 xv, u32x4 wv, float (&d)[HK]) {
  if constexpr (DT == DT_F32) {
    const f32x4 x = __builtin_bit_cast(f32x4, xv), w = __builtin_bit_cast(f32x4, wv);
    d[0] += x.x * w.x; d[1] += x.y * w.y; d[2] += x.z * w.z; d[3] += x.w * w.w;
  } else if constexpr (DT == DT_F16) {
    const f16x8 x = __builtin_bit_cast(f16x8, xv), w = __builtin_bit_cast(f16x8, wv);
#pragma unroll
    for (int j = 0; j < HK; ++j) d[j] += (float)x[j] * (float)w[j];
  } else {
    const uint32_t xs[4] = {xv.x, xv.y, xv.z, xv.w}, ws[4] = {wv.x, wv.y, wv.z, wv.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      d[2 * j] += __uint_as_float(xs[j] << 16) * __uint_as_float(ws[j] << 16);
      d[2 * j + 1] += __uint_as_float(xs[j] & 0xffff0000u) * __uint_as_float(ws[j] & 0xffff0000u);
    }
  }
}

template <int DT, int NOB, int NPW>
__global__ __launch_bounds__(256) void ir_block_kernel(IrArgs a) {
  extern __shared__ __align__(16) char lds[];
  constexpr bool F32 = DT == DT_F32;
  constexpr int ES = F32 ? 4 : 2;       // storage bytes per element
  constexpr int KSTEP = F32 ? 8 : 16;   // K per operand read (both lane halves)
  constexpr int HK = KSTEP / 2;         // K elements in one lane's 16 bytes
  constexpr int EC = IR_EC;             // expanded channels per chunk
  constexpr int NKS = EC / KSTEP;       // projection K steps per chunk
  constexpr int RPE = EC * ES + 16;     // expanded-chunk LDS row pitch
  // Loads in flight per thread in the copy loops: batching them costs more
  // registers than it saves in latency -- the kernel is occupancy-bound.
  constexpr int LB = 1;                 // weights
  constexpr int LBX = 1;                // input tile

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6, l32 = lane & 31, lh = lane >> 5;

  // Weight slots: resident -> the whole E (chunk c at channel 32c); streamed
  // -> two slots of one chunk each (chunk c in slot c & 1).
  const uint32_t WR = a.resident ? a.E : 2 * EC;
  char *XL = lds + a.lds_x;    // [NPI*32][RPX]   input tile
  char *XeL = lds + a.lds_xe;  // [NPI*32][RPE]   expanded chunk
  char *WeL = lds + a.lds_we;  // [WR][RPX]       expand weights, K contiguous
  char *WpL = lds + a.lds_wp;  // [CO][RPW]       project weights, K contiguous
  char *WdL = lds + a.lds_wd;  // [9][WR]         depthwise weights (storage dtype)
  float *BeL = reinterpret_cast<float *>(lds + a.lds_b);  // [WR]
  float *BdL = BeL + WR;                                   // [WR]
  float *BpL = BdL + WR;                                   // [CO]
  const uint32_t RPX = a.C * ES + 16, RPW = WR * ES + 16;
  const uint32_t NVX = a.C * ES / 16;     // 16-byte vectors per input pixel
  const uint32_t nchunks = a.E / EC;
  const uint32_t nks_e = a.C / KSTEP;
  const uint32_t HPIX = a.HH * a.HW;
  const uint32_t TPIX = a.TH * a.TW;
  const Act act_e = act_params(a.act_e), act_d = act_params(a.act_d), act_p = act_params(a.act_p);
  auto slot = [&](uint32_t c) -> uint32_t { return a.resident ? c * EC : (c & 1) * EC; };

  const uint32_t blk = xcd_remap(blockIdx.x, gridDim.x);
  const uint32_t t_begin = (uint32_t)(((uint64_t)blk * a.ntiles) / gridDim.x);
  const uint32_t t_end = (uint32_t)(((uint64_t)(blk + 1) * a.ntiles) / gridDim.x);
  if (t_begin >= t_end) return;

  const char *xg = reinterpret_cast<const char *>(a.x);
  const char *weg = reinterpret_cast<const char *>(a.we);
  const char *wpg = reinterpret_cast<const char *>(a.wp);

  // ---- weights of chunk c (channels [32c, 32c + 32)) -> weight slot s --------
  // Packed 1x1 weights hold element (k, n) at (k/4 * Nn + n) * 4 + k%4
  // (pack.rs:95 with one tap), so HK consecutive K of one output channel are
  // one (fp32) or two (16-bit) vectors of 4.
  auto ld_we = [&](uint32_t c, uint32_t i) -> u32x4 {  // item i = (kq, e)
    const uint32_t kq = i / EC, e = i - kq * EC;
    if constexpr (F32) {
      return *reinterpret_cast<const u32x4 *>(weg + ((size_t)kq * a.E + c * EC + e) * 16);
    } else {
      const u32x2 lo = *reinterpret_cast<const u32x2 *>(weg + ((size_t)(2 * kq) * a.E + c * EC + e) * 8);
      const u32x2 hi = *reinterpret_cast<const u32x2 *>(weg + ((size_t)(2 * kq + 1) * a.E + c * EC + e) * 8);
      return u32x4{lo.x, lo.y, hi.x, hi.y};
    }
  };
  auto st_we = [&](uint32_t s, uint32_t i, u32x4 v) {
    const uint32_t kq = i / EC, e = i - kq * EC;
    *reinterpret_cast<u32x4 *>(WeL + (s + e) * RPX + kq * 16) = v;
  };
  auto ld_wp = [&](uint32_t c, uint32_t i) -> u32x4 {  // item i = (kq, o)
    const uint32_t kq = fdiv(i, a.fd_co), o = i - kq * a.CO;
    const uint32_t kg = c * (EC / 4) + kq * (HK / 4);
    if constexpr (F32) {
      return *reinterpret_cast<const u32x4 *>(wpg + ((size_t)kg * a.CO + o) * 16);
    } else {
      const u32x2 lo = *reinterpret_cast<const u32x2 *>(wpg + ((size_t)kg * a.CO + o) * 8);
      const u32x2 hi = *reinterpret_cast<const u32x2 *>(wpg + ((size_t)(kg + 1) * a.CO + o) * 8);
      return u32x4{lo.x, lo.y, hi.x, hi.y};
    }
  };
  auto st_wp = [&](uint32_t s, uint32_t i, u32x4 v) {
    const uint32_t kq = fdiv(i, a.fd_co), o = i - kq * a.CO;
    *reinterpret_cast<u32x4 *>(WpL + o * RPW + (s + kq * HK) * ES) = v;
  };
  // Small per-chunk tensors, EC/4 vec4 per row: rows 0..8 depthwise weights
  // and row 9 its bias travel with the projection part; row 10, the expand
  // bias, travels with the expand part.
  constexpr int NSMALL_P = 10 * (EC / 4), NSMALL_E = EC / 4;
  auto ld_small = [&](uint32_t c, uint32_t row, uint32_t g) -> u32x4 {
    if (row < 9) {
      const size_t vi = (size_t)row * (a.E / 4) + c * (EC / 4) + g;
      if constexpr (F32) return reinterpret_cast<const u32x4 *>(a.wd)[vi];
      const u32x2 h = reinterpret_cast<const u32x2 *>(a.wd)[vi];
      return u32x4{h.x, h.y, 0u, 0u};
    }
    return __builtin_bit_cast(u32x4, Vec4IO<DT>::load(row == 9 ? a.bd : a.be, c * (EC / 4) + g));  // fp32
  };
  auto st_small = [&](uint32_t s, uint32_t row, uint32_t g, u32x4 v) {
    if (row < 9) {
      char *dst = WdL + ((size_t)row * WR + s + 4 * g) * ES;
      if constexpr (F32)
        *reinterpret_cast<u32x4 *>(dst) = v;
      else
        *reinterpret_cast<u32x2 *>(dst) = u32x2{v.x, v.y};
    } else {
      *reinterpret_cast<u32x4 *>((row == 9 ? BdL : BeL) + s + 4 * g) = v;
    }
  };
  const uint32_t nwe = EC * (a.C / HK), nwp = a.CO * (EC / HK);
  // synchronous load of chunk c's weights (batched so the loads overlap)
  auto load_chunk = [&](uint32_t c, bool expand_part, bool project_part) {
    const uint32_t s = slot(c);
    if (expand_part) {
      for (uint32_t i0 = tid; i0 < nwe; i0 += 256 * LB) {
        u32x4 v[LB];
#pragma unroll
        for (int b = 0; b < LB; ++b)
          if (i0 + 256 * b < nwe) v[b] = ld_we(c, i0 + 256 * b);
#pragma unroll
        for (int b = 0; b < LB; ++b)
          if (i0 + 256 * b < nwe) st_we(s, i0 + 256 * b, v[b]);
      }
    }
    if (project_part) {
      for (uint32_t i0 = tid; i0 < nwp; i0 += 256 * LB) {
        u32x4 v[LB];
#pragma unroll
        for (int b = 0; b < LB; ++b)
          if (i0 + 256 * b < nwp) v[b] = ld_wp(c, i0 + 256 * b);
#pragma unroll
        for (int b = 0; b < LB; ++b)
          if (i0 + 256 * b < nwp) st_wp(s, i0 + 256 * b, v[b]);
      }
      if (tid < NSMALL_P) st_small(s, tid / (EC / 4), tid % (EC / 4), ld_small(c, tid / (EC / 4), tid % (EC / 4)));
    }
    if (expand_part && tid < NSMALL_E) st_small(s, 10, tid, ld_small(c, 10, tid));
  };

  for (uint32_t i = tid; i < a.CO / 4; i += 256)
    *reinterpret_cast<f32x4 *>(BpL + 4 * i) = Vec4IO<DT>::load(a.bp, i);
  if (a.resident)
    for (uint32_t c = 0; c < nchunks; ++c) load_chunk(c, true, true);

  for (uint32_t T = t_begin; T < t_end; ++T) {
    const uint32_t per_img = a.tiles_y * a.tiles_x;
    const uint32_t img = fdiv(T, a.fd_pi);
    const uint32_t trem = T - img * per_img;
    const uint32_t tyi = fdiv(trem, a.fd_tx);
    const uint32_t ty0 = tyi * a.TH, tx0 = (trem - tyi * a.tiles_x) * a.TW;
    const int32_t iy0 = (int32_t)(ty0 * a.S) - a.PT, ix0 = (int32_t)(tx0 * a.S) - a.PL;
    const size_t img_px = (size_t)img * a.IH * a.IW;

    // every wavefront is done with the previous tile's LDS
    __syncthreads();
    // (0) input tile with halo -> XL (zero outside the image), and for
    // streamed weights the first chunks: expand of 0 and 1, projection of 0
    {
      const uint32_t nitems = a.NPI * 32 * NVX;
      for (uint32_t i0 = tid; i0 < nitems; i0 += 256 * LBX) {
        u32x4 val[LBX];
        uint32_t dst[LBX];
#pragma unroll
        for (int b = 0; b < LBX; ++b) {
          const uint32_t i = i0 + 256 * b;
          if (i < nitems) {
            const uint32_t r = fdiv(i, a.fd_nvx), v = i - r * NVX;
            const uint32_t hy = fdiv(r, a.fd_hw), hx = r - hy * a.HW;
            const int32_t iy = iy0 + (int32_t)hy, ix = ix0 + (int32_t)hx;
            dst[b] = r * RPX + v * 16;
            val[b] = u32x4{};
            if (r < HPIX && (uint32_t)iy < a.IH && (uint32_t)ix < a.IW)
              val[b] = *reinterpret_cast<const u32x4 *>(xg + (img_px + (size_t)iy * a.IW + ix) * a.C * ES + v * 16);
          }
        }
#pragma unroll
        for (int b = 0; b < LBX; ++b)
          if (i0 + 256 * b < nitems) *reinterpret_cast<u32x4 *>(XL + dst[b]) = val[b];
      }
    }
    if (!a.resident) load_chunk(0, true, true);
    __syncthreads();

    // tap row offsets (bytes, buffer 0) of this wavefront's output pixel blocks
    uint32_t rowo[NPW][9];
    bool live[NPW];
#pragma unroll
    for (int i = 0; i < NPW; ++i) {
      const uint32_t pbo = wave + 4 * i;
      live[i] = pbo < a.NPB;
      const uint32_t op = pbo * 32 + l32;
      const bool valid = live[i] && op < TPIX;
      const uint32_t oy = valid ? fdiv(op, a.fd_tw) : 0;
      const uint32_t ox = valid ? op - oy * a.TW : 0;
      const uint32_t base = oy * a.S * a.HW + ox * a.S;
#pragma unroll
      for (int t = 0; t < 9; ++t) rowo[i][t] = (base + (t / 3) * a.HW + t % 3) * RPE + lh * 16;
    }

    // (1) expand chunk c over the halo tile -> XeL
    auto expand = [&](uint32_t c) {
      const uint32_t ws = slot(c);
      char *xe = XeL;
      for (uint32_t b = wave; b < a.NPI; b += 4) {
        const char *ap = WeL + (ws + l32) * RPX + lh * 16;
        const char *bp = XL + (b * 32 + l32) * RPX + lh * 16;
        f32x16 acc = {};
        u32x4 a0 = *reinterpret_cast<const u32x4 *>(ap), b0 = *reinterpret_cast<const u32x4 *>(bp);
        for (uint32_t ks = 0; ks < nks_e; ++ks) {
          u32x4 a1 = a0, b1 = b0;
          if (ks + 1 < nks_e) {
            a1 = *reinterpret_cast<const u32x4 *>(ap + (ks + 1) * 32);
            b1 = *reinterpret_cast<const u32x4 *>(bp + (ks + 1) * 32);
          }
          acc = ir_mma<DT>(a0, b0, acc);
          a0 = a1;
          b0 = b1;
        }
        const uint32_t r = b * 32 + l32;
        const uint32_t hy = fdiv(r, a.fd_hw), hx = r - hy * a.HW;
        const int32_t iy = iy0 + (int32_t)hy, ix = ix0 + (int32_t)hx;
        const bool inside = r < HPIX && (uint32_t)iy < a.IH && (uint32_t)ix < a.IW;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const uint32_t el = 8 * q + 4 * lh;
          float v[4] = {acc[4 * q], acc[4 * q + 1], acc[4 * q + 2], acc[4 * q + 3]};
          const f32x4 bb = *reinterpret_cast<const f32x4 *>(BeL + ws + el);
          v[0] += bb.x; v[1] += bb.y; v[2] += bb.z; v[3] += bb.w;
          act_array<4>(act_e, v);
          if (!inside) v[0] = v[1] = v[2] = v[3] = 0.0f;
          if constexpr (F32)
            *reinterpret_cast<f32x4 *>(xe + r * RPE + el * 4) = f32x4{v[0], v[1], v[2], v[3]};
          else
            *reinterpret_cast<u32x2 *>(xe + r * RPE + el * 2) = pack4<DT>(f32x4{v[0], v[1], v[2], v[3]});
        }
      }
    };

    f32x16 acc[NPW][NOB];
#pragma unroll
    for (int i = 0; i < NPW; ++i)
#pragma unroll
      for (int o = 0; o < NOB; ++o) acc[i][o] = f32x16{};

    // Chunk loop: expand(c) | barrier | depthwise + project(c), then the next
    // chunk's streamed weights into the other slot | barrier.
    for (uint32_t c = 0; c < nchunks; ++c) {
      expand(c);
      __syncthreads();

      // (2) depthwise of chunk c straight into the projection's B operand;
      // the wavefront's pixel blocks share every K step's weight reads
      {
        const uint32_t ws = slot(c);
        const char *xe = XeL;
        const char *wdp = WdL + ws * ES + lh * 16;
        const uint32_t wd_row = WR * ES;
        const float *bdp = BdL + ws + lh * HK;
        const char *wpp = WpL + l32 * RPW + ws * ES + lh * 16;
        // one K step at a time: hoisting the next step's 18 operand reads
        // above this one doubles the live registers and halves occupancy
#pragma unroll 1
        for (int ks = 0; ks < NKS; ++ks) {
          u32x4 wv[9];
#pragma unroll
          for (int t = 0; t < 9; ++t) wv[t] = *reinterpret_cast<const u32x4 *>(wdp + t * wd_row + ks * 32);
          float bias[HK];
#pragma unroll
          for (int j = 0; j < HK; j += 4) {
            const f32x4 bb = *reinterpret_cast<const f32x4 *>(bdp + ks * KSTEP + j);
            bias[j] = bb.x; bias[j + 1] = bb.y; bias[j + 2] = bb.z; bias[j + 3] = bb.w;
          }
          u32x4 bop[NPW];
#pragma unroll
          for (int i = 0; i < NPW; ++i) {
            if (!live[i]) continue;
            float d[HK];
#pragma unroll
            for (int j = 0; j < HK; ++j) d[j] = bias[j];
#pragma unroll
            for (int t = 0; t < 9; ++t)
              ir_fma_taps<DT, HK>(*reinterpret_cast<const u32x4 *>(xe + rowo[i][t] + ks * 32), wv[t], d);
            act_array<HK>(act_d, d);
            bop[i] = ir_pack<DT, HK>(d);
          }
#pragma unroll
          for (int o = 0; o < NOB; ++o) {
            const u32x4 av = *reinterpret_cast<const u32x4 *>(wpp + o * 32 * RPW + ks * 32);
#pragma unroll
            for (int i = 0; i < NPW; ++i)
              if (live[i]) acc[i][o] = ir_mma<DT>(av, bop[i], acc[i][o]);
          }
        }
      }

      // the other slot held chunk c - 1, whose depthwise finished before this
      // chunk's expand
      if (!a.resident && c + 1 < nchunks) load_chunk(c + 1, true, true);
      __syncthreads();
    }

    // epilogue: bias -> act -> (+ residual) -> HBM
#pragma unroll
    for (int i = 0; i < NPW; ++i) {
      const uint32_t pbo = wave + 4 * i;
      if (pbo >= a.NPB) continue;
      const uint32_t op = pbo * 32 + l32;
      const uint32_t oy = fdiv(op, a.fd_tw), ox = op - oy * a.TW;
      const uint32_t gy = ty0 + oy, gx = tx0 + ox;
      if (op >= TPIX || gy >= a.OH || gx >= a.OW) continue;
      const size_t pix = ((size_t)img * a.OH + gy) * a.OW + gx;
#pragma unroll
      for (int o = 0; o < NOB; ++o) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const uint32_t oc = o * 32 + 8 * q + 4 * lh;
          f32x4 v = f32x4{acc[i][o][4 * q], acc[i][o][4 * q + 1], acc[i][o][4 * q + 2], acc[i][o][4 * q + 3]} +
                    *reinterpret_cast<const f32x4 *>(BpL + oc);
          v = act4(act_p, v);
          const size_t vi = pix * (a.CO / 4) + oc / 4;
          if (a.has_res) v += Vec4IO<DT>::load(a.res, vi);
          Vec4IO<DT>::store(a.y, vi, v);
        }
      }
    }
  }
}

// The kernel may use up to the device's whole LDS (160 KB on gfx950).
template <int DT, int NOB, int NPW>
inline hipError_t ir_prepare_inst() {
  static const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void *>(ir_block_kernel<DT, NOB, NPW>),
                                                  hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
  return e;
}

template <int DT, int NOB, int NPW>
inline hipError_t ir_launch_inst(const IrArgs &a, uint32_t lds, uint32_t grid, hipStream_t st) {
  hipError_t e = ir_prepare_inst<DT, NOB, NPW>();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL((ir_block_kernel<DT, NOB, NPW>), dim3(grid), dim3(256), lds, st, a);
  return hipGetLastError();
}

// Workgroups per CU for this instantiation at `lds` bytes of dynamic LDS
// (registers and LDS both counted by the runtime).
template <int DT, int NOB, int NPW>
inline int ir_occ_inst(uint32_t lds) {
  if (ir_prepare_inst<DT, NOB, NPW>() != hipSuccess) return 0;
  int per_cu = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, ir_block_kernel<DT, NOB, NPW>, 256, lds) != hipSuccess)
    return 0;
  return per_cu;
}

// Dispatch on the projection width (NOB = CO / 32 output-channel blocks) and
// the output pixel blocks per wavefront (NPW).
template <int DT>
inline hipError_t ir_launch_dt(const IrArgs &a, uint32_t lds, uint32_t grid, hipStream_t st) {
  const uint32_t nob = a.CO / 32, npw = (a.NPB + 3) / 4;
  switch (nob * 4 + npw) {
    case 1 * 4 + 1: return ir_launch_inst<DT, 1, 1>(a, lds, grid, st);
    case 1 * 4 + 2: return ir_launch_inst<DT, 1, 2>(a, lds, grid, st);
    case 2 * 4 + 1: return ir_launch_inst<DT, 2, 1>(a, lds, grid, st);
    case 2 * 4 + 2: return ir_launch_inst<DT, 2, 2>(a, lds, grid, st);
    case 3 * 4 + 1: return ir_launch_inst<DT, 3, 1>(a, lds, grid, st);
    case 3 * 4 + 2: return ir_launch_inst<DT, 3, 2>(a, lds, grid, st);
    case 4 * 4 + 1: return ir_launch_inst<DT, 4, 1>(a, lds, grid, st);
    case 4 * 4 + 2: return ir_launch_inst<DT, 4, 2>(a, lds, grid, st);
    default: return hipErrorInvalidValue;
  }
}

template <int DT>
inline int ir_occ_dt(uint32_t nob, uint32_t npw, uint32_t lds) {
  switch (nob * 4 + npw) {
    case 1 * 4 + 1: return ir_occ_inst<DT, 1, 1>(lds);
    case 1 * 4 + 2: return ir_occ_inst<DT, 1, 2>(lds);
    case 2 * 4 + 1: return ir_occ_inst<DT, 2, 1>(lds);
    case 2 * 4 + 2: return ir_occ_inst<DT, 2, 2>(lds);
    case 3 * 4 + 1: return ir_occ_inst<DT, 3, 1>(lds);
    case 3 * 4 + 2: return ir_occ_inst<DT, 3, 2>(lds);
    case 4 * 4 + 1: return ir_occ_inst<DT, 4, 1>(lds);
    case 4 * 4 + 2: return ir_occ_inst<DT, 4, 2>(lds);
    default: return 0;
  }
}

hipError_t launch_ir_block_f32(const IrArgs &a, uint32_t lds, uint32_t grid, hipStream_t st);
hipError_t launch_ir_block_f16(const IrArgs &a, uint32_t lds, uint32_t grid, hipStream_t st);
hipError_t launch_ir_block_bf16(const IrArgs &a, uint32_t lds, uint32_t grid, hipStream_t st);
int ir_occ_f32(uint32_t nob, uint32_t npw, uint32_t lds);
int ir_occ_f16(uint32_t nob, uint32_t npw, uint32_t lds);
int ir_occ_bf16(uint32_t nob, uint32_t npw, uint32_t lds);

}  // namespace aih
