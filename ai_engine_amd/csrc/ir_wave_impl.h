// ir_wave_impl.h -- fused inverted-residual block, one output tile per
// wavefront (16-bit storage, clamp-type activations).
//
// The same three convs as ir_block_impl.h (1x1 expand + act, depthwise 3x3
// stride S + act, 1x1 project + act (+ residual); crates/ai-gpu-runtime/src/
// lowering.rs:122-152 dispatches them separately) with the same arithmetic
// and rounding points, decomposed for overlap instead of sharing:
//
//   * every wavefront owns its own output tile of at most 32 pixels (one
//     MFMA column block) and runs expand -> depthwise -> project for it
//     alone; its expanded chunk lives in a private LDS region, so the
//     wavefronts of a workgroup never wait for each other between phases --
//     while one is in its MFMA expand another runs its VALU depthwise;
//   * the input tile (with its halo, NPI blocks of 32 pixels) goes from
//     memory straight into MFMA operand registers once per tile (16-byte
//     buffer loads, zeros outside the image through the range check) and
//     is reused by every chunk;
//   * the expand / project / depthwise weights of a 32-channel chunk sit in
//     LDS in the converter's packed layouts (pack.rs:68-122), shared by the
//     workgroup: all chunks resident for the whole launch when they fit (no
//     workgroup barrier after the first), else streamed through two slots,
//     the next chunk's copy (LDS-direct loads) overlapping the current one,
//     with one barrier per chunk.
//
// MFMA convention as in ir_block_impl.h: weights are the A operand (rows =
// channels), pixels the B operand, v_mfma_f32_32x32x16_{f16,bf16}; lane l
// holds pixel l%32 and channels 8*(r/4) + 4*(l/32) + r%4 of a result. The
// expand bias enters as one extra K step against a column that is 1.0 for
// pixels inside the image and 0 outside, so outside pixels expand to exactly
// 0 (the depthwise zero padding; the activations here are all clamp-type,
// act(0) = 0). The depthwise of the K slice a lane feeds to the projection
// is computed by that lane (fp32 accumulation, v_fma_mix / v_dot2c), so its
// result is the projection's B operand without an LDS round trip.
#pragma once

#include "ir_block_impl.h"

namespace aih {

// Global -> LDS copy of n items of SZ bytes (LDS-direct loads, no
// registers): item g from byte offset src(g) + soff (soff: a wavefront-
// uniform part, added in the scalar offset); the workgroup's `threads`
// take 64-item rows in turn, a row per wavefront. Asynchronous until
// ir_dma_wait() and a barrier.
template <int SZ, class F>
__device__ __forceinline__ void irw_dma(char *dst, uint32_t n, __amdgpu_buffer_rsrc_t rs, int wave, int lane,
                                        uint32_t threads, F src, uint32_t soff = 0) {
  for (uint32_t g0 = (uint32_t)wave * 64; g0 < n; g0 += threads) {
    const uint32_t g = g0 + lane;
    if (g >= n) continue;
    ir_lds_void *d = (ir_lds_void *)(dst + g0 * SZ);
    if constexpr (SZ == 16)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, d, 16, src(g), (int)soff, 0, 0);
    else
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, d, 4, src(g), (int)soff, 0, 0);
  }
}

// ReLU of two 16-bit floats packed in 32 bits, as 16-bit signed integers:
// every negative float (and -0) has its sign bit set, so max(bits, 0) is 0
// exactly where max(x, 0) is, and a non-negative float keeps its bits (one
// v_pk_max_i16 for two values). Rounding is monotone and keeps the sign, so
// relu(round(x)) == round(relu(x)) bit for bit: packing first is exact.
__device__ __forceinline__ uint32_t irw_relu2(uint32_t v) {
  typedef short s16x2 __attribute__((ext_vector_type(2)));
  return __builtin_bit_cast(uint32_t, __builtin_elementwise_max(__builtin_bit_cast(s16x2, v), s16x2{0, 0}));
}

// act(v) rounded to the storage dtype, 4 values -> 8 bytes: ReLU after the
// conversion on packed 16-bit integers; other clamp-type activations before
// it (one v_med3_f32 each).
template <int DT, bool RELU>
__device__ __forceinline__ u32x2 irw_act_pack4(const Act &p, f32x4 v) {
  if constexpr (RELU) {
    const u32x2 b = pack4<DT>(v);
    return u32x2{irw_relu2(b.x), irw_relu2(b.y)};
  }
  float t[4] = {v.x, v.y, v.z, v.w};
  ir_act<true, 4>(p, t);
  return pack4<DT>(f32x4{t[0], t[1], t[2], t[3]});
}

// Orders this wavefront's LDS accesses on either side (its lanes write the
// expanded chunk that other lanes of the same wavefront read next; a
// wavefront's LDS operations complete in issue order, so only the compiler
// must not move them across).
__device__ __forceinline__ void irw_wave_order() {
  __builtin_amdgcn_sched_barrier(0);
  asm volatile("" ::: "memory");
}

// KE: expand K steps (C / 16); NPI: 32-pixel blocks of the halo tile; NOB:
// projection blocks of 32 output channels; RL: the expand and depthwise
// activations are both ReLU (applied to the packed 16-bit results).
template <int DT, int KE, int NPI, int NOB, bool RL>
__global__ __launch_bounds__(IRW_THREADS) void ir_wave_kernel(IrWaveArgs a) {
  static_assert(DT == DT_F16 || DT == DT_BF16, "16-bit storage");
  extern __shared__ __align__(16) char lds[];
  constexpr int ES = 2, KSTEP = 16, HK = 8, EC = 32, NKS = EC / KSTEP;
  constexpr uint32_t GB = 4 * ES;  // one packed group: 4 K of one channel
  constexpr uint32_t C = KE * KSTEP;
  constexpr uint32_t WES = EC * C * ES;  // expand weights of one chunk
  // depthwise taps whose operands are read in one batch: all nine when the
  // registers held across a chunk (input halo, expand A operands, projection
  // accumulators) leave room for 72 more, else one row of three. The
  // narrowest shape (HELD <= 64) fits four waves per SIMD in 128 VGPRs only
  // with the short batch; four waves beat the long one there.
  constexpr int HELD = 4 * NPI * KE + 4 * KE + 16 * NOB;
  constexpr int TB = HELD > 64 && HELD <= 120 ? 9 : 3;
  // packed ReLU where the registers allow it (it keeps the packed results
  // live longer; the widest instantiations would spill): on the expand's
  // epilogue (RLE) and the depthwise result (RLD) -- on the narrowest shape
  // only the former keeps it within 128 VGPRs
  constexpr bool RLE = RL && HELD <= 130;
  constexpr bool RLD = RL && HELD > 64 && HELD <= 130;
  const int tid = threadIdx.x;
  const int lane = tid & 63, l32 = lane & 31, lh = lane >> 5;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  // wavefronts of this workgroup (2, 4 or 8, chosen by the plan)
  const uint32_t nthr = blockDim.x, nwaves = nthr >> 6;

  const uint32_t WPG = EC * a.CO * ES;         // project weights of one chunk in memory
  const uint32_t WPS = EC * a.COP * ES;        // ... in a slot, rows padded to COP channels
  const uint32_t SLOT = WES + WPS + IRW_SMB;   // 16-byte multiple (C, COP multiples of 16 / 32)
  const uint32_t nchunks = a.E / EC;
  char *WL = lds + a.lds_w;
  float *BpL = reinterpret_cast<float *>(lds + a.lds_bp);
  char *XeL = lds + a.lds_xe + (uint32_t)wave * (NPI * 32 * IRW_RPE);
  const Act act_e = act_params(a.act_e), act_d = act_params(a.act_d), act_p = act_params(a.act_p);

  const __amdgpu_buffer_rsrc_t rs_we = ir_rsrc(a.we, C * a.E * ES);
  const __amdgpu_buffer_rsrc_t rs_wp = ir_rsrc(a.wp, a.E * a.CO * ES);
  const __amdgpu_buffer_rsrc_t rs_wd = ir_rsrc(a.wd, 9 * a.E * ES);
  const __amdgpu_buffer_rsrc_t rs_bd = ir_rsrc(a.bd, a.E * ES);
  const __amdgpu_buffer_rsrc_t rs_be = ir_rsrc(a.be, a.E * ES);

  // chunk c's weights (expanded channels [32c, 32c + 32)) -> slot s, byte
  // for byte in the packed layouts: expand element (k, e) at (k/4 * E + e) * 4
  // + k%4 gives C/4 runs of 32 channels; the project weights of K rows
  // [32c, 32c + 32) are one contiguous run (EC/4 runs of CO channels, each
  // to a COP-channel row when CO < COP); depthwise taps 9 runs of 32.
  auto dma_chunk = [&](uint32_t c, uint32_t s) {
    char *slot = WL + s * SLOT;
    constexpr uint32_t GR = EC * GB / 16;  // 16-byte items per expand run
    irw_dma<16>(slot, (C / 4) * GR, rs_we, wave, lane, nthr,
                [&](uint32_t g) -> uint32_t { return ((g / GR) * a.E + EC * c) * GB + (g % GR) * 16; });
    if (a.COP == a.CO) {
      irw_dma<16>(slot + WES, WPS / 16, rs_wp, wave, lane, nthr,
                  [&](uint32_t g) -> uint32_t { return c * WPG + g * 16; });
    } else {
      const uint32_t rb = a.CO * GB;  // bytes of one K group's run
      for (uint32_t q = 0; q < EC / 4; ++q)
        irw_dma<16>(slot + WES + q * (a.COP * GB), rb / 16, rs_wp, (wave + q) % nwaves, lane, nthr,
                    [&](uint32_t g) -> uint32_t { return c * WPG + q * rb + g * 16; });
    }
    constexpr uint32_t TR = EC * ES / 16;  // 16-byte items per depthwise tap run
    char *sm = slot + WES + WPS;
    irw_dma<16>(sm, 9 * TR, rs_wd, wave, lane, nthr,
                [&](uint32_t g) -> uint32_t { return ((g / TR) * a.E + EC * c) * ES + (g % TR) * 16; });
    irw_dma<4>(sm + 9 * EC * ES, EC * ES / 4, rs_bd, wave, lane, nthr,
               [&](uint32_t g) -> uint32_t { return EC * c * ES + g * 4; });
    irw_dma<4>(sm + 10 * EC * ES, EC * ES / 4, rs_be, wave, lane, nthr,
               [&](uint32_t g) -> uint32_t { return EC * c * ES + g * 4; });
  };

  for (uint32_t i = tid; i < a.CO / 4; i += nthr)
    *reinterpret_cast<f32x4 *>(BpL + 4 * i) = Vec4IO<DT>::load(a.bp, i);
  if (a.COP != a.CO) {
    // project weights of channels CO..COP: zero in every slot, for good (the
    // copies write only channels below CO)
    const uint32_t nslots = a.resident ? nchunks : 2u, pad16 = (a.COP - a.CO) * GB / 16;
    for (uint32_t i = tid; i < nslots * (EC / 4) * pad16; i += nthr) {
      const uint32_t sq = i / pad16, v = i - sq * pad16;
      *reinterpret_cast<u32x4 *>(WL + (sq / (EC / 4)) * SLOT + WES + (sq % (EC / 4)) * (a.COP * GB) + a.CO * GB +
                                 v * 16) = u32x4{0u, 0u, 0u, 0u};
    }
  }
  if (a.resident) {
    for (uint32_t c = 0; c < nchunks; ++c) dma_chunk(c, c);
  } else {
    dma_chunk(0, 0);
  }
  ir_dma_wait();
  __syncthreads();
  constexpr bool BSPLIT = DT == DT_BF16 && irw_bf16_split(KE, NPI, NOB);
  if constexpr (BSPLIT) {
    if (a.resident) {
      // every chunk's depthwise taps split by channel parity, once: the
      // slot keeps the even channels (odd halves zeroed), lds_hi gets the
      // odd ones (even halves zeroed)
      constexpr uint32_t TW = 9 * EC / 2;  // 32-bit words of one chunk's taps
      for (uint32_t i = tid; i < nchunks * TW; i += nthr) {
        const uint32_t c = i / TW, r = i - c * TW;
        uint32_t *wlo = reinterpret_cast<uint32_t *>(WL + c * SLOT + WES + WPS) + r;
        const uint32_t w = *wlo;
        *wlo = w & 0x0000ffffu;
        reinterpret_cast<uint32_t *>(lds + a.lds_hi + c * IRW_HI_BYTES)[r] = w & 0xffff0000u;
      }
      __syncthreads();
    }
  }

  // this workgroup's contiguous range of tiles (handed out XCD by XCD)
  const uint32_t blk = xcd_remap(blockIdx.x, gridDim.x, a.nxcd);
  const uint32_t t_begin = (uint32_t)(((uint64_t)blk * a.ntiles) / gridDim.x);
  const uint32_t t_end = (uint32_t)(((uint64_t)(blk + 1) * a.ntiles) / gridDim.x);

  const char *xg = reinterpret_cast<const char *>(a.x);
  const uint32_t img_bytes = a.IH * a.IW * C * ES;
  const uint32_t per_img = a.tiles_y * a.tiles_x;
  const uint32_t HPIX = a.HH * a.HW, TPIX = a.TH * a.TW;
  constexpr uint32_t ONE = DT == DT_F16 ? 0x3C00u : 0x3F80u;

  // ---- per-tile state of this wavefront ----
  u32x4 xop[NPI][KE];  // input halo pixels as expand B operands
  bool inside[NPI];    // this lane's halo pixel of block b lies in the image
  uint32_t rowo[3];    // LDS byte offsets of this lane's three depthwise tap rows
  size_t out_pix = 0;  // this lane's output pixel
  bool out_ok = false;
  f32x16 acc[NOB];

  auto begin_tile = [&](uint32_t T) {
    const uint32_t img = fdiv(T, a.fd_pi);
    const uint32_t trem = T - img * per_img;
    const uint32_t tyi = fdiv(trem, a.fd_tx);
    const uint32_t ty0 = tyi * a.TH, tx0 = (trem - tyi * a.tiles_x) * a.TW;
    const int32_t iy0 = (int32_t)(ty0 * a.S) - a.PT, ix0 = (int32_t)(tx0 * a.S) - a.PL;
    const __amdgpu_buffer_rsrc_t rs_x = ir_rsrc(xg + (size_t)img * img_bytes, img_bytes);
#pragma unroll
    for (int b = 0; b < NPI; ++b) {
      const uint32_t r = b * 32 + l32;
      const uint32_t hy = fdiv(r, a.fd_hw), hx = r - hy * a.HW;
      const int32_t iy = iy0 + (int32_t)hy, ix = ix0 + (int32_t)hx;
      const bool in = r < HPIX && (uint32_t)iy < a.IH && (uint32_t)ix < a.IW;
      const uint32_t off = in ? ((uint32_t)iy * a.IW + (uint32_t)ix) * (C * ES) + lh * 16 : IR_OOB;
#pragma unroll
      for (int k = 0; k < KE; ++k)
        xop[b][k] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs_x, off + k * 32, 0, 0));
      inside[b] = in;
    }
    const uint32_t op = l32;
    const bool in_tile = op < TPIX;
    const uint32_t oy = in_tile ? fdiv(op, a.fd_tw) : 0, ox = in_tile ? op - oy * a.TW : 0;
    const uint32_t base = oy * a.S * a.HW + ox * a.S;
#pragma unroll
    for (int dy = 0; dy < 3; ++dy) rowo[dy] = (base + dy * a.HW) * IRW_RPE + lh * 16;
    const uint32_t gy = ty0 + oy, gx = tx0 + ox;
    out_ok = in_tile && gy < a.OH && gx < a.OW;
    out_pix = ((size_t)img * a.OH + gy) * a.OW + gx;
#pragma unroll
    for (int o = 0; o < NOB; ++o) acc[o] = f32x16{};
  };

  // expand of chunk `slot` over the halo tile -> this wavefront's XeL, then
  // its depthwise + projection into acc; hi: the chunk's odd-channel taps
  // (bf16 with resident weights, the slot's taps then hold the even ones),
  // else null
  auto run_chunk = [&](const char *slot, const char *hi) {
    // expand A operands of the chunk: channel l32, K groups from 2 * lh; a K
    // step advances 4 groups of 32 channels (1024 bytes)
    const char *ap = slot + ((uint32_t)lh * (HK / 4) * EC + l32) * GB;
    u32x4 aw[KE];
#pragma unroll
    for (int k = 0; k < KE; ++k) aw[k] = ir_ld_w<DT>(ap + k * (KSTEP * EC * ES), EC * GB);
    const char *sm = slot + WES + WPS;
    const uint32_t bw = lh == 0 ? (uint32_t)*reinterpret_cast<const uint16_t *>(sm + 10 * EC * ES + l32 * 2) : 0u;
#pragma unroll
    for (int b = 0; b < NPI; ++b) {
      const u32x4 bx = {(lh == 0 && inside[b]) ? ONE : 0u, 0u, 0u, 0u};
      f32x16 e = ir_mma<DT>(u32x4{bw, 0u, 0u, 0u}, bx, f32x16{});
#pragma unroll
      for (int k = 0; k < KE; ++k) e = ir_mma<DT>(aw[k], xop[b][k], e);
      char *row = XeL + (b * 32 + l32) * IRW_RPE;
#pragma unroll
      for (int q = 0; q < 4; ++q)
        *reinterpret_cast<u32x2 *>(row + (8 * q + 4 * lh) * ES) =
            irw_act_pack4<DT, RLE>(act_e, f32x4{e[4 * q], e[4 * q + 1], e[4 * q + 2], e[4 * q + 3]});
    }
    irw_wave_order();

    const char *wdp = sm + lh * 16;                 // tap t at + t * EC * ES
    const char *bdp = sm + 9 * EC * ES + lh * 16;
    const char *wpp = slot + WES + ((uint32_t)lh * (HK / 4) * a.COP + l32) * GB;
    const uint32_t wp_ks = KSTEP / 4 * a.COP * GB, wp_next = a.COP * GB;
#pragma unroll 1
    for (int ks = 0; ks < NKS; ++ks) {
      // the operands of TB taps go out together (2 * TB reads in flight),
      // then their FMAs; all nine at once where the registers allow
      float d[HK];
      ir_unpack<DT, HK>(*reinterpret_cast<const u32x4 *>(bdp + ks * 32), d);
#pragma unroll
      for (int t0 = 0; t0 < 9; t0 += TB) {
        u32x4 wv[TB], xv[TB];
#pragma unroll
        for (int t = 0; t < TB; ++t) wv[t] = *reinterpret_cast<const u32x4 *>(wdp + (t0 + t) * (EC * ES) + ks * 32);
#pragma unroll
        for (int t = 0; t < TB; ++t)
          xv[t] = *reinterpret_cast<const u32x4 *>(XeL + rowo[(t0 + t) / 3] + ((t0 + t) % 3) * IRW_RPE + ks * 32);
        if constexpr (BSPLIT) {
          if (hi) {
            u32x4 wh[TB];
#pragma unroll
            for (int t = 0; t < TB; ++t)
              wh[t] = *reinterpret_cast<const u32x4 *>(hi + lh * 16 + (t0 + t) * (EC * ES) + ks * 32);
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int t = 0; t < TB; ++t) ir_fma_taps_bf16_split<HK>(xv[t], wv[t], wh[t], d);
            continue;
          }
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int t = 0; t < TB; ++t) ir_fma_taps<DT, HK>(xv[t], wv[t], d);
      }
      u32x4 bop;
      if constexpr (RLD) {
        bop = ir_pack<DT, HK>(d);
        bop = u32x4{irw_relu2(bop.x), irw_relu2(bop.y), irw_relu2(bop.z), irw_relu2(bop.w)};
      } else {
        ir_act<true, HK>(act_d, d);
        bop = ir_pack<DT, HK>(d);
      }
#pragma unroll
      for (int o = 0; o < NOB; ++o)
        acc[o] = ir_mma<DT>(ir_ld_w<DT>(wpp + o * (32 * GB) + ks * wp_ks, wp_next), bop, acc[o]);
      __builtin_amdgcn_sched_barrier(0);
    }
    // the next chunk's expand overwrites XeL after these reads
    irw_wave_order();
  };

  auto end_tile = [&]() {
    if (!out_ok) return;
#pragma unroll
    for (int o = 0; o < NOB; ++o) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const uint32_t oc = o * 32 + 8 * q + 4 * lh;
        if (o == NOB - 1 && oc >= a.CO) continue;  // padding channels of the last block
        f32x4 v = f32x4{acc[o][4 * q], acc[o][4 * q + 1], acc[o][4 * q + 2], acc[o][4 * q + 3]} +
                  *reinterpret_cast<const f32x4 *>(BpL + oc);
        float t4[4] = {v.x, v.y, v.z, v.w};
        ir_act<true, 4>(act_p, t4);
        v = f32x4{t4[0], t4[1], t4[2], t4[3]};
        const size_t vi = out_pix * (a.CO / 4) + oc / 4;
        if (a.has_res) v += Vec4IO<DT>::load(a.res, vi);
        Vec4IO<DT>::store(a.y, vi, v);
      }
    }
  };

  if (a.resident) {
    // every chunk in LDS: the wavefronts run their tiles independently
    for (uint32_t T = t_begin + wave; T < t_end; T += nwaves) {
      begin_tile(T);
      for (uint32_t c = 0; c < nchunks; ++c)
        run_chunk(WL + c * SLOT, BSPLIT ? lds + a.lds_hi + c * IRW_HI_BYTES : nullptr);
      end_tile();
    }
    return;
  }

  // streamed weights: the wavefronts walk the chunks in step (one barrier a
  // chunk), chunk number gc of the workgroup's run in slot gc & 1; the next
  // chunk's copy goes out as soon as every wavefront is done with its slot
  uint32_t gc = 0;
  for (uint32_t T0 = t_begin; T0 < t_end; T0 += nwaves) {
    const uint32_t T = T0 + wave;
    const bool active = T < t_end;  // wave-uniform
    const bool more = T0 + nwaves < t_end;
    if (active) begin_tile(T);
    for (uint32_t c = 0; c < nchunks; ++c, ++gc) {
      // chunk gc has landed (every wavefront's share) and slot (gc + 1) & 1
      // is free: every wavefront finished chunk gc - 1
      ir_dma_wait();
      __syncthreads();
      const bool last = c + 1 == nchunks;
      if (!last || more) dma_chunk(last ? 0 : c + 1, (gc + 1) & 1);
      if (active) run_chunk(WL + (gc & 1) * SLOT, nullptr);
    }
    if (active) end_tile();
  }
  ir_dma_wait();
}

template <int DT, int KE, int NPI, int NOB, bool RL>
inline hipError_t irw_prepare_inst() {
  static const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void *>(ir_wave_kernel<DT, KE, NPI, NOB, RL>),
                                                  hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
  return e;
}

template <int DT, int KE, int NPI, int NOB, bool RL>
inline hipError_t irw_launch_inst(const IrWaveArgs &a, uint32_t waves, uint32_t lds, uint32_t grid, hipStream_t st) {
  const hipError_t e = irw_prepare_inst<DT, KE, NPI, NOB, RL>();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL((ir_wave_kernel<DT, KE, NPI, NOB, RL>), dim3(grid), dim3(64 * waves), lds, st, a);
  return hipGetLastError();
}

template <int DT, int KE, int NPI, int NOB, bool RL>
inline int irw_occ_inst(uint32_t waves, uint32_t lds) {
  if (irw_prepare_inst<DT, KE, NPI, NOB, RL>() != hipSuccess) return -1;
  int per_cu = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, ir_wave_kernel<DT, KE, NPI, NOB, RL>, (int)(64 * waves),
                                                   lds) != hipSuccess)
    return -1;
  return per_cu;
}

// The (KE, NPI, NOB) combinations with an instantiation: the inverted-residual
// blocks of the MobileNet-style encoders (C = 16 KE input channels, NPI halo
// blocks: 2 for a stride-1 tile of <= 32 pixels, 5 for stride 2, NOB = COP /
// 32) and the 48 -> 96 -> 48 blocks of the converter's segmentation model.
#define AIH_IRW_SHAPES(X) X(2, 2, 1) X(2, 5, 2) X(3, 2, 2) X(4, 2, 2) X(4, 5, 3) X(6, 2, 3) X(8, 2, 4)

inline bool irw_has_shape(uint32_t ke, uint32_t npi, uint32_t nob) {
#define AIH_IRW_HAS(KE, NPI, NOB) \
  if (ke == KE && npi == NPI && nob == NOB) return true;
  AIH_IRW_SHAPES(AIH_IRW_HAS)
#undef AIH_IRW_HAS
  return false;
}

// Both inner activations ReLU: the instantiation that applies them to packed results.
inline bool irw_relu_inner(int act_e, int act_d) { return act_e == AIH_ACT_RELU && act_d == AIH_ACT_RELU; }

template <int DT>
inline hipError_t irw_launch_dt(const IrWaveArgs &a, uint32_t npi, uint32_t waves, uint32_t lds, uint32_t grid,
                                hipStream_t st) {
  const uint32_t ke = a.C / 16, nob = a.COP / 32;
  const bool rl = irw_relu_inner(a.act_e, a.act_d);
#define AIH_IRW_LAUNCH(KE, NPI, NOB)                                                          \
  if (ke == KE && npi == NPI && nob == NOB)                                                   \
    return rl ? irw_launch_inst<DT, KE, NPI, NOB, true>(a, waves, lds, grid, st)             \
              : irw_launch_inst<DT, KE, NPI, NOB, false>(a, waves, lds, grid, st);
  AIH_IRW_SHAPES(AIH_IRW_LAUNCH)
#undef AIH_IRW_LAUNCH
  return hipErrorInvalidValue;
}

template <int DT>
inline int irw_occ_dt(uint32_t ke, uint32_t npi, uint32_t nob, bool rl, uint32_t waves, uint32_t lds) {
#define AIH_IRW_OCC(KE, NPI, NOB)                                                                        \
  if (ke == KE && npi == NPI && nob == NOB)                                                              \
    return rl ? irw_occ_inst<DT, KE, NPI, NOB, true>(waves, lds) : irw_occ_inst<DT, KE, NPI, NOB, false>(waves, lds);
  AIH_IRW_SHAPES(AIH_IRW_OCC)
#undef AIH_IRW_OCC
  return 0;
}

hipError_t launch_ir_wave_f16(const IrWaveArgs &a, uint32_t npi, uint32_t waves, uint32_t lds, uint32_t grid,
                              hipStream_t st);
hipError_t launch_ir_wave_bf16(const IrWaveArgs &a, uint32_t npi, uint32_t waves, uint32_t lds, uint32_t grid,
                               hipStream_t st);
int ir_wave_occ_f16(uint32_t ke, uint32_t npi, uint32_t nob, bool rl, uint32_t waves, uint32_t lds);
int ir_wave_occ_bf16(uint32_t ke, uint32_t npi, uint32_t nob, bool rl, uint32_t waves, uint32_t lds);

}  // namespace aih
