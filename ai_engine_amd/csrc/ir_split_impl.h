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
//     meet in LDS (with eight wavefronts, 4 + w first added to w, so the
//     region holds four), and the wavefront that owns an output block adds
//     them in wavefront order (a fixed order: the result does not depend on
//     timing) before the bias, activation, residual and store.
//
// Projection channels CO..COP (cout not a multiple of 32) read zero weights
// through the buffer range check and are never stored.
#pragma once

#include "conv_pw_narrow.h"
#include "ir_wave_impl.h"

namespace aih {

template <int DT, int KE, int NPI, int NOB, bool RL, bool DP>
__global__ __launch_bounds__(IRW_THREADS) void ir_split_kernel(IrWaveArgs a) {
  static_assert(DT == DT_F16 || DT == DT_BF16, "16-bit storage");
  extern __shared__ __align__(16) char lds[];
  constexpr int ES = 2, EC = 32, NOG = 2 * NOB;
  constexpr uint32_t GB = 4 * ES;  // one packed group: 4 K of one channel
  constexpr uint32_t C = KE * 16;
  // Registers held across a chunk: the expand operands, the accumulators and
  // the projection operands. The projection operands go out before the
  // expand where the shape stays within 128 VGPRs (four wavefronts per
  // SIMD), else after it. The packed ReLU on the expand's epilogue and on
  // the depthwise result.
  constexpr int HELD = 4 * KE + 16 * NOB + 8 * NOB;
  constexpr bool RLE = RL, RLD = RL;
  constexpr bool WP_EARLY = HELD <= 64;
  const int tid = threadIdx.x;
  const int lane = tid & 63, l32 = lane & 31, lh = lane >> 5, l16 = lane & 15, q = lane >> 4;
  const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const uint32_t nw = blockDim.x >> 6;
  const uint32_t nchunks = a.E / EC;
  const uint32_t c_begin = wave * nchunks / nw, c_end = (wave + 1) * nchunks / nw;

  float *BpL = reinterpret_cast<float *>(lds + a.lds_bp);
  f32x4 *HeadL = reinterpret_cast<f32x4 *>(lds + a.lds_head);
  constexpr uint32_t RPX = C * ES + 16;  // halo row pitch: the pixel's C channels + 16 bytes
  const char *XL = lds + a.lds_x;
  constexpr uint32_t PLANE = NPI * 32 * 16;  // one 8-channel plane of the expanded chunk
  char *XeL = lds + a.lds_xe + wave * (4 * PLANE);
  // ring slot s of this wavefront at SmL + s * IRW_SMB (the slot layout of
  // the wave kernel: 9 taps, zero run, depthwise bias, expand bias)
  char *SmL = lds + a.lds_w + wave * (2 * IRW_SMB);
  const Act act_e = act_params(a.act_e), act_d = act_params(a.act_d), act_p = act_params(a.act_p);
  const IrDwLane DL = irdw_lane(lane);

  const __amdgpu_buffer_rsrc_t rs_we = ir_rsrc(a.we, C * a.E * ES);
  const __amdgpu_buffer_rsrc_t rs_wp = ir_rsrc(a.wp, a.E * a.CO * ES);
  const __amdgpu_buffer_rsrc_t rs_wd = ir_rsrc(a.wd, 9 * a.E * ES);
  const __amdgpu_buffer_rsrc_t rs_bd = ir_rsrc(a.bd, a.E * ES);
  const __amdgpu_buffer_rsrc_t rs_be = ir_rsrc(a.be, a.E * ES);

  for (uint32_t i = tid; i < a.CO / 4; i += blockDim.x)
    *reinterpret_cast<f32x4 *>(BpL + 4 * i) = Vec4IO<DT>::load(a.bp, i);
  // the zero run of this wavefront's two ring slots (its copies never write it)
  if (lane < 8)
    *reinterpret_cast<u32x4 *>(SmL + (lane >> 2) * IRW_SMB + IRW_TAPS_ZERO + (lane & 3) * 16) =
        u32x4{0u, 0u, 0u, 0u};

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
  // this lane's output pixel of each 16-pixel group and its depthwise B offsets in XeL
  uint32_t bc[2][3], br[2], pix[2];
  bool ok[2];
#pragma unroll
  for (int pg = 0; pg < 2; ++pg) {
    const uint32_t op = pg * 16 + l16;
    const bool in_tile = op < TPIX;
    const uint32_t oy = in_tile ? fdiv(op, a.fd_tw) : 0, ox = in_tile ? op - oy * a.TW : 0;
    irdw_rows(oy * a.S * a.HW + ox * a.S, a.HW, q, PLANE, bc[pg], br[pg]);
    ok[pg] = in_tile && ty0 + oy < a.OH && tx0 + ox < a.OW;
    pix[pg] = (img * a.OH + ty0 + oy) * a.OW + tx0 + ox;
  }

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
  // projection A operands of chunk c: block og, output channel 16 og + l16,
  // K slice q = packed groups 8c + q and 8c + q + 4 (the depthwise result's
  // K order); zeros for channels CO..COP (a lane offset past every buffer)
  auto load_wp = [&](uint32_t c, u32x4 (&wp)[NOG]) {
    const uint32_t so = 8 * c * a.CO * GB;
#pragma unroll
    for (int og = 0; og < NOG; ++og) {
      const uint32_t ch = (uint32_t)og * 16 + l16;
      const uint32_t vo = ch < a.CO ? ((uint32_t)q * a.CO + ch) * GB : IR_OOB;
      const u32x2 lo = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(rs_wp, vo, so, 0));
      const u32x2 hi = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(rs_wp, vo, so + 4 * a.CO * GB, 0));
      wp[og] = u32x4{lo.x, lo.y, hi.x, hi.y};
    }
  };
  // depthwise taps, depthwise bias, expand bias of chunk c -> ring slot s;
  // this wavefront's LDS-direct loads, landed at its next ir_dma_wait
  auto load_small = [&](uint32_t c, uint32_t s) {
    char *sm = SmL + s * IRW_SMB;
    constexpr uint32_t TR = EC * ES / 16;  // 16-byte items per tap run
    irw_dma<16>(sm, 9 * TR, rs_wd, 0, lane, 64,
                [&](uint32_t g) -> uint32_t { return (g / TR) * a.E * ES + (g % TR) * 16; }, EC * c * ES);
    irw_dma<4>(sm + IRW_BD, EC * ES / 4, rs_bd, 0, lane, 64, [&](uint32_t g) -> uint32_t { return g * 4; },
               EC * c * ES);
    irw_dma<4>(sm + IRW_BE, EC * ES / 4, rs_be, 0, lane, 64, [&](uint32_t g) -> uint32_t { return g * 4; },
               EC * c * ES);
  };

  f32x4 acc[NOG][2];
#pragma unroll
  for (int og = 0; og < NOG; ++og) acc[og][0] = acc[og][1] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

  // expand of the chunk whose small tensors are at sm, over the halo tile ->
  // XeL, each K step's B operands read from LDS one step ahead. With the deep
  // prefetch (registers to spare) the halo blocks go two at a time with their
  // MFMA chains interleaved (two accumulators), so an MFMA does not wait for
  // the one before it.
  constexpr int G = DP ? 2 : 1;
  auto expand = [&](const char *sm, const u32x4 (&aw)[KE]) {
    const uint32_t bw = lh == 0 ? (uint32_t)*reinterpret_cast<const uint16_t *>(sm + IRW_BE + l32 * 2) : 0u;
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
        // channels 8 qq + 4 lh .. + 3: plane qq, the pixel's 16 bytes at 8 lh
        char *px = XeL + ((b0 + g) * 32 + l32) * 16 + lh * 8;
#pragma unroll
        for (int qq = 0; qq < 4; ++qq)
          *reinterpret_cast<u32x2 *>(px + qq * PLANE) = irw_act_pack4<DT, RLE>(
              act_e, f32x4{e[g][4 * qq], e[g][4 * qq + 1], e[g][4 * qq + 2], e[g][4 * qq + 3]});
      }
    }
  };
  // depthwise of the chunk at sm (expanded rows in XeL) and its projection
  // into acc with operands wpv
  auto dw_project = [&](const char *sm, const u32x4 (&wpv)[NOG]) {
    u32x4 bop[2];
    irdw_chunk<DT, RLD, PLANE>(XeL, sm, DL, bc, br, q, act_d, bop);
#pragma unroll
    for (int og = 0; og < NOG; ++og) {
      if (og * 16 >= (int)a.CO) continue;
#pragma unroll
      for (int pg = 0; pg < 2; ++pg) acc[og][pg] = ir_mma16<DT>(wpv[og], bop[pg], acc[og][pg]);
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
      char *sm = SmL + s * IRW_SMB;
      // chunk c's small tensors have landed (and every earlier load)
      ir_dma_wait();
      irw_wave_order();
      // the projection operands (in flight during the expand where registers allow)
      u32x4 wpv[NOG];
      if constexpr (WP_EARLY) load_wp(c, wpv);

      expand(sm, aw);
      irw_wave_order();
      // the next chunk's operands go out now: its expand weights into the
      // registers this expand has finished with, its small tensors into the
      // other ring slot (last read by the previous chunk, whose reads are done)
      if (c + 1 < c_end) {
        load_aw(c + 1, aw);
        load_small(c + 1, s ^ 1u);
      }
      if constexpr (!WP_EARLY) load_wp(c, wpv);
      dw_project(sm, wpv);
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
      char *sm = SmL + s * IRW_SMB;
      ir_dma_wait();
      irw_wave_order();
      u32x4 wpv[NOG];
      load_wp(c, wpv);
      if (c + 1 < c_end) {
        load_aw(c + 1, nxt);
        load_small(c + 1, s ^ 1u);
      }
      expand(sm, cur);
      irw_wave_order();
      dw_project(sm, wpv);
      irw_wave_order();
    };
    for (uint32_t c = c_begin; c < c_end; c += 2) {
      step(c, 0, awA, awB);
      if (c + 1 < c_end) step(c + 1, 1, awB, awA);
    }
  }

  // ---- partial sums: slot s's unit (og, pg) at [s][og][pg][lane] (f32x4) ----
  // The region overlaps the halo, the wavefronts' XeL and rings: every
  // wavefront must be done with them first. At most four slots: with eight
  // wavefronts, 4..7 first pass theirs to 0..3, which add them to their own
  // (so the region holds four wavefronts' sums, not eight).
  __syncthreads();
  f32x4 *red = reinterpret_cast<f32x4 *>(lds + a.lds_red);
  const uint32_t nslot = nw < 4 ? nw : 4;
  if (nw > 4) {
    if (wave >= 4) {
#pragma unroll
      for (int og = 0; og < NOG; ++og)
#pragma unroll
        for (int pg = 0; pg < 2; ++pg) red[(((wave - 4) * NOG + og) * 2 + pg) * 64 + lane] = acc[og][pg];
    }
    __syncthreads();
    if (wave < 4) {
#pragma unroll
      for (int og = 0; og < NOG; ++og)
#pragma unroll
        for (int pg = 0; pg < 2; ++pg) acc[og][pg] += red[((wave * NOG + og) * 2 + pg) * 64 + lane];
    }
    __syncthreads();
  }
  if (wave < nslot) {
#pragma unroll
    for (int og = 0; og < NOG; ++og)
#pragma unroll
      for (int pg = 0; pg < 2; ++pg) red[((wave * NOG + og) * 2 + pg) * 64 + lane] = acc[og][pg];
  }
  __syncthreads();
  // unit u = (og, pg) belongs to wavefront u % W: the sum over the slots in
  // order (a fixed order: the result does not depend on timing), then bias ->
  // act -> (+ residual) -> store
  for (uint32_t u = wave; u < (uint32_t)(2 * NOG); u += nw) {
    const uint32_t og = u >> 1, pg = u & 1;
    const uint32_t oc = og * 16 + 4 * q;
    // (selects, not a register array indexed at run time)
    const bool okp = pg ? ok[1] : ok[0];
    const uint32_t pixp = pg ? pix[1] : pix[0];
    if (og * 16 >= a.CO || !okp) continue;  // padding channels of the last block; pixels outside
    f32x4 v = red[((0 * NOG + og) * 2 + pg) * 64 + lane];
    for (uint32_t s = 1; s < nslot; ++s) v += red[((s * NOG + og) * 2 + pg) * 64 + lane];
    v += *reinterpret_cast<const f32x4 *>(BpL + oc);
    float t4[4] = {v.x, v.y, v.z, v.w};
    ir_act<true, 4>(act_p, t4);
    v = f32x4{t4[0], t4[1], t4[2], t4[3]};
    const size_t vi = (size_t)pixp * (a.CO / 4) + oc / 4;
    if (a.has_res) v += Vec4IO<DT>::load(a.res, vi);
    if (a.y) Vec4IO<DT>::store(a.y, vi, v);
    if (a.hy) {
      // the joined head: pw_narrow_kernel's lane g = kg % 16 of this pixel
      // sums input groups g, g + 16, ... in that order, starting from 0; this
      // unit holds group kg = oc / 4 (the same wavefront runs kg + 16 after
      // kg, units u and u + 8), its four outputs added to lane g's slot. The
      // inputs are the block's outputs as stored (rounded to DT).
      const f32x4 xr = unpack4<DT>(pack4<DT>(v));
      const uint32_t kg = oc / 4;
      f32x4 *slot = HeadL + (pg * 16 + l16) * 16 + (kg & 15);
      f32x4 d;
#pragma unroll
      for (int j = 0; j < 4; ++j) d[j] = narrow_dot4(xr, narrow_w4<DT, DT>(a.hw, (size_t)kg * 4 + j));
      *slot = (kg < 16 ? f32x4{0.0f, 0.0f, 0.0f, 0.0f} : *slot) + d;
    }
  }
  if (a.hy) {
    // lane pg * 16 + p of wavefront 0 finishes pixel p of group pg: the
    // 16 lanes' sums added as pw_narrow_kernel's butterfly leaves them in
    // its lane 0 (xor 8, 4, 2, 1), then bias -> act -> store
    __syncthreads();
    if (wave == 0 && lane < 32) {
      const uint32_t pg = (uint32_t)lane >> 4;
      const bool okp = pg ? ok[1] : ok[0];
      const uint32_t pixp = pg ? pix[1] : pix[0];
      const f32x4 *P = HeadL + lane * 16;
      f32x4 s8[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) s8[i] = P[i] + P[i + 8];
      const f32x4 t0 = s8[0] + s8[4], t1 = s8[1] + s8[5], t2 = s8[2] + s8[6], t3 = s8[3] + s8[7];
      const f32x4 acc_h = (t0 + t2) + (t1 + t3);
      const f32x4 hb = Vec4IO<DT>::load(a.hb, 0);
      float v[4] = {acc_h.x + hb.x, acc_h.y + hb.y, acc_h.z + hb.z, acc_h.w + hb.w};
      act_array<4>(act_params(a.act_h), v);
      if (okp) Vec4IO<DT>::store(a.hy, pixp, f32x4{v[0], v[1], v[2], v[3]});
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
