// ir_split_impl.h -- fused inverted-residual block for launches with few
// output tiles: the wavefronts of a workgroup share one output tile and split
// its expanded channels (16-bit storage, clamp-type activations).
//
// The late blocks of a MobileNet-style encoder have a small image (10x18 or
// 20x36 outputs) and a wide expansion (E = 256..512): a few hundred to a few
// thousand 32-pixel tiles, against 1024 SIMDs. With one tile per wavefront
// (ir_wave_impl.h) most SIMDs hold one wavefront or none, and its weights
// (100..300 KB) are streamed through LDS with a workgroup barrier per chunk.
// Here a workgroup of W wavefronts takes one tile, and wavefront w runs the
// expand -> depthwise -> project chain of ir_wave_impl.h for the chunks
// [w * nchunks / W, (w + 1) * nchunks / W) only; W x more wavefronts carry the
// same work. The chain's arithmetic is that of the wave kernel; what differs:
//
//   * the tile's input halo is copied to LDS once for the workgroup (LDS-
//     direct loads, zeros outside the image) and every wavefront reads its
//     expand B operands from there, chunk by chunk: no halo held in
//     registers, so more wavefronts fit on a SIMD;
//   * no weight is shared through LDS, so no barrier is taken after the
//     halo's until the end:
//     the expand and projection A operands go from memory (L2: every tile
//     reads the same weights) straight into registers -- a chunk's
//     projection operands before its expand (or, for the widest blocks,
//     before each K step's depthwise), the next chunk's expand
//     operands while the current chunk runs its depthwise -- and the chunk's
//     depthwise taps and biases into a private two-slot LDS ring (LDS-direct
//     loads, completed by the wavefront's own wait);
//   * each wavefront ends with projection partial sums over its chunks. They
//     meet in LDS, and the wavefront that owns an output block adds the W
//     partials in wavefront order (a fixed order: the result does not depend
//     on timing) before the bias, activation, residual and store.
//
// Projection channels CO..COP (cout not a multiple of 32) read zero weights
// through the buffer range check and are never stored.
#pragma once

#include "ir_wave_impl.h"

namespace aih {

template <int DT, int KE, int NPI, int NOB, bool RL, bool DP>
__global__ __launch_bounds__(IRW_THREADS) void ir_split_kernel(IrWaveArgs a) {
  static_assert(DT == DT_F16 || DT == DT_BF16, "16-bit storage");
  extern __shared__ __align__(16) char lds[];
  constexpr int ES = 2, KSTEP = 16, HK = 8, EC = 32, NKS = EC / KSTEP;
  constexpr uint32_t GB = 4 * ES;  // one packed group: 4 K of one channel
  constexpr uint32_t C = KE * KSTEP;
  // Registers held across a chunk: the expand operands, the accumulators and
  // both K steps' projection operands. Depthwise taps are read in batches of
  // three; the projection operands go out before the expand where the shape
  // stays within 128 VGPRs (four wavefronts per SIMD), else before each K
  // step's depthwise. The packed ReLU on the expand's epilogue only: on the
  // depthwise result it keeps the packed values live longer and costs a
  // wavefront per SIMD on the wider shapes.
  constexpr int HELD = 4 * KE + 16 * NOB + 8 * NOB;
  constexpr int TB = 3;
  constexpr bool RLE = RL, RLD = false;
  constexpr bool WP_EARLY = HELD <= 64;
  const int tid = threadIdx.x;
  const int lane = tid & 63, l32 = lane & 31, lh = lane >> 5;
  const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const uint32_t nw = blockDim.x >> 6;
  const uint32_t nchunks = a.E / EC;
  const uint32_t c_begin = wave * nchunks / nw, c_end = (wave + 1) * nchunks / nw;

  float *BpL = reinterpret_cast<float *>(lds + a.lds_bp);
  constexpr uint32_t RPX = C * ES + 16;  // halo row pitch: the pixel's C channels + 16 bytes
  const char *XL = lds + a.lds_x;
  char *XeL = lds + a.lds_xe + wave * (NPI * 32 * IRW_RPE);
  // ring slot s of this wavefront at SmL + s * SMS; BS (bf16 on the narrow
  // shapes): the slot's taps split by channel parity (split_taps), the odd
  // halves IRW_SMB bytes in
  constexpr bool BS = DT == DT_BF16 && irs_bf16_split(KE, NPI);
  constexpr uint32_t SMS = BS ? IRS_SLOT_BF16 : IRW_SMB;
  char *SmL = lds + a.lds_w + wave * (2 * SMS);
  const Act act_e = act_params(a.act_e), act_d = act_params(a.act_d), act_p = act_params(a.act_p);

  const __amdgpu_buffer_rsrc_t rs_we = ir_rsrc(a.we, C * a.E * ES);
  const __amdgpu_buffer_rsrc_t rs_wp = ir_rsrc(a.wp, a.E * a.CO * ES);
  const __amdgpu_buffer_rsrc_t rs_wd = ir_rsrc(a.wd, 9 * a.E * ES);
  const __amdgpu_buffer_rsrc_t rs_bd = ir_rsrc(a.bd, a.E * ES);
  const __amdgpu_buffer_rsrc_t rs_be = ir_rsrc(a.be, a.E * ES);

  for (uint32_t i = tid; i < a.CO / 4; i += blockDim.x)
    *reinterpret_cast<f32x4 *>(BpL + 4 * i) = Vec4IO<DT>::load(a.bp, i);

  // ---- the tile: its input halo -> XL, row r = halo pixel r ----
  const uint32_t T = xcd_remap(blockIdx.x, gridDim.x, a.nxcd);
  const uint32_t per_img = a.tiles_y * a.tiles_x;
  const uint32_t img = fdiv(T, a.fd_pi);
  const uint32_t trem = T - img * per_img;
  const uint32_t tyi = fdiv(trem, a.fd_tx);
  const uint32_t ty0 = tyi * a.TH, tx0 = (trem - tyi * a.tiles_x) * a.TW;
  const uint32_t HPIX = a.HH * a.HW, TPIX = a.TH * a.TW;
  const int32_t iy0 = (int32_t)(ty0 * a.S) - a.PT, ix0 = (int32_t)(tx0 * a.S) - a.PL;
  constexpr uint32_t ONE = DT == DT_F16 ? 0x3C00u : 0x3F80u;
  {
    const uint32_t img_bytes = a.IH * a.IW * C * ES;
    const __amdgpu_buffer_rsrc_t rs_x =
        ir_rsrc(reinterpret_cast<const char *>(a.x) + (size_t)img * img_bytes, img_bytes);
    constexpr uint32_t NV = C * ES / 16;  // 16-byte items per pixel; item NV of a row is its padding
    irw_dma<16>(const_cast<char *>(XL), NPI * 32 * (NV + 1), rs_x, (int)wave, lane, blockDim.x,
                [&](uint32_t g) -> uint32_t {
                  const uint32_t r = g / (NV + 1), v = g - r * (NV + 1);
                  const uint32_t hy = fdiv(r, a.fd_hw), hx = r - hy * a.HW;
                  const int32_t iy = iy0 + (int32_t)hy, ix = ix0 + (int32_t)hx;
                  const bool in = v < NV && r < HPIX && (uint32_t)iy < a.IH && (uint32_t)ix < a.IW;
                  return in ? ((uint32_t)iy * a.IW + (uint32_t)ix) * (C * ES) + v * 16 : IR_OOB;
                });
  }
  // this lane's halo pixel of block b lies in the image (its expand bias column)
  bool inside[NPI];
#pragma unroll
  for (int b = 0; b < NPI; ++b) {
    const uint32_t r = b * 32 + l32;
    const uint32_t hy = fdiv(r, a.fd_hw), hx = r - hy * a.HW;
    const int32_t iy = iy0 + (int32_t)hy, ix = ix0 + (int32_t)hx;
    inside[b] = r < HPIX && (uint32_t)iy < a.IH && (uint32_t)ix < a.IW;
  }
  // this lane's output pixel and its three depthwise tap rows in XeL
  const bool in_tile = (uint32_t)l32 < TPIX;
  const uint32_t oy = in_tile ? fdiv(l32, a.fd_tw) : 0, ox = in_tile ? l32 - oy * a.TW : 0;
  uint32_t rowo[3];
#pragma unroll
  for (int dy = 0; dy < 3; ++dy) rowo[dy] = ((oy * a.S + dy) * a.HW + ox * a.S) * IRW_RPE + lh * 16;
  const bool out_ok = in_tile && ty0 + oy < a.OH && tx0 + ox < a.OW;
  const size_t out_pix = ((size_t)img * a.OH + ty0 + oy) * a.OW + tx0 + ox;

  // ---- weights of chunk c ----
  // Every weight offset is a lane part (held) plus a wavefront-uniform part
  // that goes into the buffer load's scalar offset (no per-chunk address
  // arithmetic on the vector unit).
  // expand A operands: channel 32c + l32, K groups 4k + 2 lh and the next
  // (packed element (k, e) at (k/4 * E + e) * 4 + k%4)
  const uint32_t vo_aw = ((uint32_t)lh * 2 * a.E + l32) * GB;
  auto load_aw = [&](uint32_t c, u32x4 (&aw)[KE]) {
#pragma unroll
    for (int k = 0; k < KE; ++k) {
      const uint32_t so = (EC * c + (uint32_t)k * 4 * a.E) * GB;
      const u32x2 lo = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(rs_we, vo_aw, so, 0));
      const u32x2 hi = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(rs_we, vo_aw, so + a.E * GB, 0));
      aw[k] = u32x4{lo.x, lo.y, hi.x, hi.y};
    }
  };
  // projection A operand of block o, K step ks: output channel 32o + l32, K
  // rows 32c + 16ks + 8lh .. + 8 (groups 8c + 4ks + 2lh and the next); zeros
  // for channels CO..COP (a lane offset past every buffer)
  auto load_wp = [&](uint32_t c, int ks, int o) -> u32x4 {
    const uint32_t ch = (uint32_t)o * 32 + l32;
    const uint32_t vo = ch < a.CO ? (2 * (uint32_t)lh * a.CO + ch) * GB : IR_OOB;
    const uint32_t so = (8 * c + 4 * (uint32_t)ks) * a.CO * GB;
    const u32x2 lo = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(rs_wp, vo, so, 0));
    const u32x2 hi = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(rs_wp, vo, so + a.CO * GB, 0));
    return u32x4{lo.x, lo.y, hi.x, hi.y};
  };
  // depthwise taps, depthwise bias, expand bias of chunk c -> ring slot s
  // (9 runs of 32 channels, then the two biases: the slot layout of the wave
  // kernel); this wavefront's LDS-direct loads, landed at its next ir_dma_wait
  auto load_small = [&](uint32_t c, uint32_t s) {
    char *sm = SmL + s * SMS;
    constexpr uint32_t TR = EC * ES / 16;  // 16-byte items per tap run
    irw_dma<16>(sm, 9 * TR, rs_wd, 0, lane, 64,
                [&](uint32_t g) -> uint32_t { return (g / TR) * a.E * ES + (g % TR) * 16; }, EC * c * ES);
    irw_dma<4>(sm + 9 * EC * ES, EC * ES / 4, rs_bd, 0, lane, 64, [&](uint32_t g) -> uint32_t { return g * 4; },
               EC * c * ES);
    irw_dma<4>(sm + 10 * EC * ES, EC * ES / 4, rs_be, 0, lane, 64, [&](uint32_t g) -> uint32_t { return g * 4; },
               EC * c * ES);
  };

  // BS: ring slot sm's taps (landed, this wavefront's own) split by
  // channel parity -- even halves kept in place, odd halves IRW_SMB bytes
  // in -- so each tap is two v_dot2c with no per-use masking; the
  // wavefront's LDS accesses stay in issue order, no barrier
  auto split_taps = [&](char *sm) {
    if constexpr (BS) {
      constexpr uint32_t TW = 9 * EC / 2;  // 32-bit words of one chunk's taps
      uint32_t *lo = reinterpret_cast<uint32_t *>(sm), *hi = reinterpret_cast<uint32_t *>(sm + IRW_SMB);
#pragma unroll
      for (uint32_t i = (uint32_t)lane; i < TW; i += 64) {
        const uint32_t w = lo[i];
        lo[i] = w & 0x0000ffffu;
        hi[i] = w & 0xffff0000u;
      }
      irw_wave_order();
    }
  };

  f32x16 acc[NOB];
#pragma unroll
  for (int o = 0; o < NOB; ++o) acc[o] = f32x16{};

  auto load_wp_all = [&](uint32_t c, u32x4 (&wp)[NKS][NOB]) {
#pragma unroll
    for (int ks = 0; ks < NKS; ++ks)
#pragma unroll
      for (int o = 0; o < NOB; ++o) wp[ks][o] = load_wp(c, ks, o);
  };
  // expand of the chunk whose small tensors are at sm, over the halo tile ->
  // XeL, each K step's B operands read from LDS one step ahead. With the deep
  // prefetch (registers to spare) the halo blocks go two at a time with their
  // MFMA chains interleaved (two accumulators), so an MFMA does not wait for
  // the one before it.
  constexpr int G = DP ? 2 : 1;
  auto expand = [&](const char *sm, const u32x4 (&aw)[KE]) {
    const uint32_t bw = lh == 0 ? (uint32_t)*reinterpret_cast<const uint16_t *>(sm + 10 * EC * ES + l32 * 2) : 0u;
#pragma unroll
    for (int b0 = 0; b0 < NPI; b0 += G) {
      const int ng = NPI - b0 < G ? NPI - b0 : G;
      f32x16 e[G];
      u32x4 xb[G][2];
      const char *xr[G];
#pragma unroll
      for (int g = 0; g < G; ++g) {
        if (g >= ng) continue;
        xr[g] = XL + ((b0 + g) * 32 + l32) * RPX + lh * 16;
        xb[g][0] = *reinterpret_cast<const u32x4 *>(xr[g]);
      }
#pragma unroll
      for (int g = 0; g < G; ++g) {
        if (g >= ng) continue;
        const u32x4 bx = {(lh == 0 && inside[b0 + g]) ? ONE : 0u, 0u, 0u, 0u};
        e[g] = ir_mma<DT>(u32x4{bw, 0u, 0u, 0u}, bx, f32x16{});
      }
#pragma unroll
      for (int k = 0; k < KE; ++k) {
#pragma unroll
        for (int g = 0; g < G; ++g)
          if (g < ng && k + 1 < KE) xb[g][(k + 1) & 1] = *reinterpret_cast<const u32x4 *>(xr[g] + (k + 1) * 32);
#pragma unroll
        for (int g = 0; g < G; ++g)
          if (g < ng) e[g] = ir_mma<DT>(aw[k], xb[g][k & 1], e[g]);
      }
#pragma unroll
      for (int g = 0; g < G; ++g) {
        if (g >= ng) continue;
        char *row = XeL + ((b0 + g) * 32 + l32) * IRW_RPE;
#pragma unroll
        for (int q = 0; q < 4; ++q)
          *reinterpret_cast<u32x2 *>(row + (8 * q + 4 * lh) * ES) = irw_act_pack4<DT, RLE>(
              act_e, f32x4{e[g][4 * q], e[g][4 * q + 1], e[g][4 * q + 2], e[g][4 * q + 3]});
      }
    }
  };

  if constexpr (!DP) {
    u32x4 aw[KE];
    if (c_begin < c_end) {
      load_aw(c_begin, aw);
      load_small(c_begin, 0);
    }
    // the halo (every wavefront's share of the copy) and the projection bias
    ir_dma_wait();
    __syncthreads();
    for (uint32_t c = c_begin; c < c_end; ++c) {
      const uint32_t s = (c - c_begin) & 1;
      char *sm = SmL + s * SMS;
      // chunk c's small tensors have landed (and every earlier load)
      ir_dma_wait();
      irw_wave_order();
      split_taps(sm);
      // the projection operands (both K steps' in flight during the expand)
      u32x4 wpv[NKS][NOB];
      if constexpr (WP_EARLY) load_wp_all(c, wpv);

      expand(sm, aw);
      irw_wave_order();
      // the next chunk's operands go out now: its expand weights into the
      // registers this expand has finished with, its small tensors into the
      // other ring slot (last read by the previous chunk, whose reads are done)
      if (c + 1 < c_end) {
        load_aw(c + 1, aw);
        load_small(c + 1, s ^ 1u);
      }

      // depthwise of the lane's K slice straight into the projection's B operand
      const char *wdp = sm + lh * 16;
      const char *bdp = sm + 9 * EC * ES + lh * 16;
#pragma unroll
      for (int ks = 0; ks < NKS; ++ks) {
        if constexpr (!WP_EARLY) {
#pragma unroll
          for (int o = 0; o < NOB; ++o) wpv[ks][o] = load_wp(c, ks, o);
        }
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
          if constexpr (BS) {
            u32x4 wh[TB];
#pragma unroll
            for (int t = 0; t < TB; ++t)
              wh[t] = *reinterpret_cast<const u32x4 *>(wdp + IRW_SMB + (t0 + t) * (EC * ES) + ks * 32);
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int t = 0; t < TB; ++t) ir_fma_taps_bf16_split<HK>(xv[t], wv[t], wh[t], d);
          } else {
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int t = 0; t < TB; ++t) ir_fma_taps<DT, HK>(xv[t], wv[t], d);
          }
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
        for (int o = 0; o < NOB; ++o) acc[o] = ir_mma<DT>(wpv[ks][o], bop, acc[o]);
        __builtin_amdgcn_sched_barrier(0);
      }
      // the next chunk's expand overwrites XeL after these reads
      irw_wave_order();
    }
  } else {
    // Deep prefetch, for launches with few wavefronts per SIMD (the
    // registers are there; other wavefronts do not hide the latency): two
    // sets of expand operands (A for the even chunks of this wavefront's run,
    // B for the odd ones) and two ring slots, so a chunk's expand weights and
    // small tensors go out at the start of the chunk before it; its
    // projection operands go out at its own start, ahead of its expand.
    u32x4 awA[KE], awB[KE];
    if (c_begin < c_end) {
      load_aw(c_begin, awA);
      load_small(c_begin, 0);
    }
    ir_dma_wait();
    __syncthreads();
    // chunk c from ring slot s with expand operands `cur`; the next chunk's
    // into `nxt` and the other slot
    auto step = [&](uint32_t c, uint32_t s, u32x4 (&cur)[KE], u32x4 (&nxt)[KE]) {
      char *sm = SmL + s * SMS;
      ir_dma_wait();
      irw_wave_order();
      split_taps(sm);
      u32x4 wpv[NKS][NOB];
#pragma unroll
      for (int ks = 0; ks < NKS; ++ks)
#pragma unroll
        for (int o = 0; o < NOB; ++o) wpv[ks][o] = load_wp(c, ks, o);
      if (c + 1 < c_end) {
        load_aw(c + 1, nxt);
        load_small(c + 1, s ^ 1u);
      }
      expand(sm, cur);
      irw_wave_order();
      const char *wdp = sm + lh * 16;
      const char *bdp = sm + 9 * EC * ES + lh * 16;
#pragma unroll
      for (int ks = 0; ks < NKS; ++ks) {
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
          if constexpr (BS) {
            u32x4 wh[TB];
#pragma unroll
            for (int t = 0; t < TB; ++t)
              wh[t] = *reinterpret_cast<const u32x4 *>(wdp + IRW_SMB + (t0 + t) * (EC * ES) + ks * 32);
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int t = 0; t < TB; ++t) ir_fma_taps_bf16_split<HK>(xv[t], wv[t], wh[t], d);
          } else {
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int t = 0; t < TB; ++t) ir_fma_taps<DT, HK>(xv[t], wv[t], d);
          }
        }
        ir_act<true, HK>(act_d, d);
        const u32x4 bop = ir_pack<DT, HK>(d);
#pragma unroll
        for (int o = 0; o < NOB; ++o) acc[o] = ir_mma<DT>(wpv[ks][o], bop, acc[o]);
        __builtin_amdgcn_sched_barrier(0);
      }
      irw_wave_order();
    };
    for (uint32_t c = c_begin; c < c_end; c += 2) {
      step(c, 0, awA, awB);
      if (c + 1 < c_end) step(c + 1, 1, awB, awA);
    }
  }

  // ---- partial sums: wavefront w's block o at [w][o][q][lane] (f32x4) ----
  // The region overlaps the halo, the wavefronts' XeL and rings: every
  // wavefront must be done with them first.
  __syncthreads();
  f32x4 *red = reinterpret_cast<f32x4 *>(lds + a.lds_red);
#pragma unroll
  for (int o = 0; o < NOB; ++o)
#pragma unroll
    for (int q = 0; q < 4; ++q)
      red[((wave * NOB + o) * 4 + q) * 64 + lane] =
          f32x4{acc[o][4 * q], acc[o][4 * q + 1], acc[o][4 * q + 2], acc[o][4 * q + 3]};
  __syncthreads();
  if (!out_ok) return;
  // block o belongs to wavefront o % W: the sum over wavefronts 0..W-1 in
  // order, then bias -> act -> (+ residual) -> store
  for (uint32_t o = wave; o < (uint32_t)NOB; o += nw) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const uint32_t oc = o * 32 + 8 * q + 4 * lh;
      if (oc >= a.CO) continue;  // padding channels of the last block
      f32x4 v = red[((0 * NOB + o) * 4 + q) * 64 + lane];
      for (uint32_t w = 1; w < nw; ++w) v += red[((w * NOB + o) * 4 + q) * 64 + lane];
      v += *reinterpret_cast<const f32x4 *>(BpL + oc);
      float t4[4] = {v.x, v.y, v.z, v.w};
      ir_act<true, 4>(act_p, t4);
      v = f32x4{t4[0], t4[1], t4[2], t4[3]};
      const size_t vi = out_pix * (a.CO / 4) + oc / 4;
      if (a.has_res) v += Vec4IO<DT>::load(a.res, vi);
      Vec4IO<DT>::store(a.y, vi, v);
    }
  }
}

template <int DT, int KE, int NPI, int NOB, bool RL, bool DP>
inline hipError_t irs_prepare_inst() {
  static const hipError_t e = hipFuncSetAttribute(
      reinterpret_cast<const void *>(ir_split_kernel<DT, KE, NPI, NOB, RL, DP>),
      hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
  return e;
}

template <int DT, int KE, int NPI, int NOB, bool RL, bool DP>
inline hipError_t irs_launch_inst(const IrWaveArgs &a, uint32_t waves, uint32_t lds, uint32_t grid,
                                  hipStream_t st) {
  const hipError_t e = irs_prepare_inst<DT, KE, NPI, NOB, RL, DP>();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL((ir_split_kernel<DT, KE, NPI, NOB, RL, DP>), dim3(grid), dim3(64 * waves), lds, st, a);
  return hipGetLastError();
}

template <int DT, int KE, int NPI, int NOB, bool RL, bool DP>
inline int irs_occ_inst(uint32_t waves, uint32_t lds) {
  if (irs_prepare_inst<DT, KE, NPI, NOB, RL, DP>() != hipSuccess) return -1;
  int per_cu = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, ir_split_kernel<DT, KE, NPI, NOB, RL, DP>,
                                                   (int)(64 * waves), lds) != hipSuccess)
    return -1;
  return per_cu;
}

template <int DT, int KE, int NPI, int NOB, bool RL>
inline hipError_t irs_launch_rl(const IrWaveArgs &a, bool deep, uint32_t waves, uint32_t lds, uint32_t grid,
                                hipStream_t st) {
  return deep ? irs_launch_inst<DT, KE, NPI, NOB, RL, true>(a, waves, lds, grid, st)
              : irs_launch_inst<DT, KE, NPI, NOB, RL, false>(a, waves, lds, grid, st);
}

template <int DT, int KE, int NPI, int NOB, bool RL>
inline int irs_occ_rl(bool deep, uint32_t waves, uint32_t lds) {
  return deep ? irs_occ_inst<DT, KE, NPI, NOB, RL, true>(waves, lds)
              : irs_occ_inst<DT, KE, NPI, NOB, RL, false>(waves, lds);
}

// The split kernel's instantiations: the wave kernel's, and the stride-2
// 96 -> 384 -> 128 block whose halo (five blocks) the wave kernel cannot hold
// in registers next to four projection blocks.
#define AIH_IRS_SHAPES(X) AIH_IRW_SHAPES(X) X(6, 5, 4)

inline bool irs_has_shape(uint32_t ke, uint32_t npi, uint32_t nob) {
#define AIH_IRS_HAS(KE, NPI, NOB) \
  if (ke == KE && npi == NPI && nob == NOB) return true;
  AIH_IRS_SHAPES(AIH_IRS_HAS)
#undef AIH_IRS_HAS
  return false;
}

template <int DT>
inline hipError_t irs_launch_dt(const IrWaveArgs &a, uint32_t npi, bool deep, uint32_t waves, uint32_t lds,
                                uint32_t grid, hipStream_t st) {
  const uint32_t ke = a.C / 16, nob = a.COP / 32;
  const bool rl = irw_relu_inner(a.act_e, a.act_d);
#define AIH_IRS_LAUNCH(KE, NPI, NOB)                                                          \
  if (ke == KE && npi == NPI && nob == NOB)                                                   \
    return rl ? irs_launch_rl<DT, KE, NPI, NOB, true>(a, deep, waves, lds, grid, st)         \
              : irs_launch_rl<DT, KE, NPI, NOB, false>(a, deep, waves, lds, grid, st);
  AIH_IRS_SHAPES(AIH_IRS_LAUNCH)
#undef AIH_IRS_LAUNCH
  return hipErrorInvalidValue;
}

template <int DT>
inline int irs_occ_dt(uint32_t ke, uint32_t npi, uint32_t nob, bool rl, bool deep, uint32_t waves, uint32_t lds) {
#define AIH_IRS_OCC(KE, NPI, NOB)                                                           \
  if (ke == KE && npi == NPI && nob == NOB)                                                 \
    return rl ? irs_occ_rl<DT, KE, NPI, NOB, true>(deep, waves, lds)                        \
              : irs_occ_rl<DT, KE, NPI, NOB, false>(deep, waves, lds);
  AIH_IRS_SHAPES(AIH_IRS_OCC)
#undef AIH_IRS_OCC
  return 0;
}

hipError_t launch_ir_split_f16(const IrWaveArgs &a, uint32_t npi, bool deep, uint32_t waves, uint32_t lds,
                               uint32_t grid, hipStream_t st);
hipError_t launch_ir_split_bf16(const IrWaveArgs &a, uint32_t npi, bool deep, uint32_t waves, uint32_t lds,
                                uint32_t grid, hipStream_t st);
int ir_split_occ_f16(uint32_t ke, uint32_t npi, uint32_t nob, bool rl, bool deep, uint32_t waves, uint32_t lds);
int ir_split_occ_bf16(uint32_t ke, uint32_t npi, uint32_t nob, bool rl, bool deep, uint32_t waves, uint32_t lds);

}  // namespace aih
